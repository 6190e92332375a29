"""The device cache end to end (bin/test_devcache.py, restated): outputs
through the cache equal the all-resident outputs EXACTLY over 40 steps at
capacities 16/32/64 of 64 experts with real shapes, eviction exercised, with
the slots in MFMA tile order (the fetch tiling the row-major host buffers as
it stores; every occupied slot holds hostpool.to_tiles of its expert) and in
row-major order, and a captured step replays DYNAMIC with the right bytes."""
import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu
E, H, I, K = 64, 2048, 512, 8


@pytest.fixture(scope="module")
def pair(dev):
    import moe
    import synth
    ref = moe.MoEExperts(E, H, I, device=dev)
    synth.fill_experts(ref, seed=0, recipe="devtest")
    host = moe.MoEExperts(E, H, I, device="cpu")
    for n in ("w13_weight", "w2_weight", "w13_scale_inv", "w2_scale_inv"):
        setattr(host, n, getattr(ref, n).cpu().pin_memory())
    return ref, host


@pytest.mark.parametrize("cap,tiles", [(16, True), (32, False), (E, True)])
def test_cache_is_bit_exact_against_resident(lib, dev, pair, cap, tiles, monkeypatch):
    import devcache
    import hipfetch
    import offload
    from fp8_moe import fp8_moe_forward
    from hostpool import to_tiles
    ref, host = pair
    monkeypatch.setattr(offload, "DEVICE_TILES", tiles)
    devcache.init_dev_cache(host, dev, cap)
    assert devcache.cache_layout(host) == (hipfetch.LAYOUT_TILES if tiles else hipfetch.LAYOUT_ROWS)
    torch.manual_seed(cap)
    say(f"devcache: capacity {cap}, tiles {tiles}")
    for step in range(40):
        x = torch.randn(1, H, device=dev).to(torch.bfloat16)
        ids = torch.randperm(E, device=dev)[:K].unsqueeze(0)
        w = torch.rand(1, K, device=dev).to(torch.bfloat16)
        w = w / w.sum(-1, keepdim=True)
        want = fp8_moe_forward(x, ids, w, ref.w13_weight, ref.w13_scale_inv, ref.w2_weight,
                               ref.w2_scale_inv)
        slots = devcache.dev_resolve_and_fetch(host, ids)
        got = fp8_moe_forward(x, slots.reshape(ids.shape), w, host._dc_w13, host._dc_s13,
                              host._dc_w2, host._dc_s2, layout=devcache.cache_layout(host))
        assert torch.equal(want, got), f"step {step}"
    occupied = int((host._dc_slot_expert >= 0).sum())
    assert occupied == cap
    order = to_tiles if tiles else (lambda t: t)
    for s_, e in enumerate(host._dc_slot_expert.tolist()):
        for c, h in ((host._dc_w13, host.w13_weight), (host._dc_w2, host.w2_weight)):
            assert torch.equal(c[s_].view(torch.uint8).cpu(), order(h[e].view(torch.uint8))), (s_, e)
        assert torch.equal(host._dc_s13[s_].cpu(), host.w13_scale_inv[e])
    hits, misses = devcache.cache_stats(host)
    assert hits + misses == 40 * K and (cap >= E or misses > cap)


@pytest.mark.parametrize("cap,wdtype", [(16, torch.bfloat16), (E, torch.float32), (9, torch.float32)])
def test_hook_fetch_ffn_is_bit_exact_against_resident(lib, dev, pair, cap, wdtype, monkeypatch):
    """dev_cached_forward through moe_resolve_fetch_ffn (the resolve made by
    the fetch launch's workgroups, the misses' gate/up run by the
    workgroups that fetch them, the hits' beside them) against the
    all-resident forward, bit for bit, and the slots' bytes in tile order."""
    import devcache
    import offload
    from fp8_moe import fp8_moe_forward
    from hostpool import to_tiles
    ref, host = pair
    monkeypatch.setattr(offload, "DEVICE_TILES", True)
    monkeypatch.setattr(devcache, "FUSED_FFN", True)
    devcache.init_dev_cache(host, dev, cap)
    torch.manual_seed(100 + cap)
    say(f"devcache fetch_ffn: capacity {cap}, weights {wdtype}")
    for step in range(40):
        x = torch.randn(1, H, device=dev).to(torch.bfloat16)
        ids = torch.randperm(E, device=dev)[:K].unsqueeze(0)
        w = torch.rand(1, K, device=dev).to(wdtype)
        w = w / w.sum(-1, keepdim=True)
        want = fp8_moe_forward(x, ids, w, ref.w13_weight, ref.w13_scale_inv, ref.w2_weight,
                               ref.w2_scale_inv)
        got = devcache.dev_cached_forward(host, x, ids, w)
        assert torch.equal(want, got), f"step {step}"
    for s_, e in enumerate(host._dc_slot_expert.tolist()):
        for c, h in ((host._dc_w13, host.w13_weight), (host._dc_w2, host.w2_weight)):
            assert torch.equal(c[s_].view(torch.uint8).cpu(), to_tiles(h[e].view(torch.uint8))), (s_, e)
        assert torch.equal(host._dc_s13[s_].cpu(), host.w13_scale_inv[e])
        assert torch.equal(host._dc_s2[s_].cpu(), host.w2_scale_inv[e])
    hits, misses = devcache.cache_stats(host)
    assert hits + misses == 40 * K and (cap >= E or misses > cap)


def _rows_with_repeats(E_, K_, n, seed):
    """Fixed rows that repeat an expert on a miss, on a hit and both in one
    row (first on a cold cache), then `n` rows drawn with replacement."""
    fixed = [[3, 3, 7, 9, 3, 11, 12, 13],       # 3 three times, all cold: a repeated miss
             [3, 9, 9, 20, 21, 22, 23, 3],      # 3 and 9 resident: repeated hits, 4 misses
             [40, 3, 40, 41, 41, 9, 42, 3]]     # repeated misses and a repeated hit
    rng = np.random.default_rng(seed)
    rows = [r[:K_] for r in fixed] + [list(rng.integers(0, E_, size=K_)) for _ in range(n)]
    return [torch.tensor([r], dtype=torch.int64) for r in rows]


@pytest.mark.parametrize("cap", [9, 16])
def test_hook_fetch_ffn_repeated_expert_in_a_row(lib, dev, pair, cap, monkeypatch):
    """A row that names an expert twice (bin/devcache.py:73-97: the second
    occurrence is a hit on the slot the first one took; a miss is queued
    once).  dev_cached_forward through moe_resolve_fetch_ffn must give every pick
    of that expert its activations, whether the expert misses or hits:
    the output equals the unfused path (resolve, fetch, forward on the
    slots) on a twin cache and the all-resident forward bit for bit, and
    the W8A8 oracle within 1e-2; the two caches' tables stay equal."""
    import devcache
    import moe
    import offload
    from fp8_moe import fp8_moe_forward
    from oracle import moe as omoe
    ref, host = pair
    twin = moe.MoEExperts(E, H, I, device="cpu")
    for n in ("w13_weight", "w2_weight", "w13_scale_inv", "w2_scale_inv"):
        setattr(twin, n, getattr(host, n))          # the same pinned tensors
    monkeypatch.setattr(offload, "DEVICE_TILES", True)
    devcache.init_dev_cache(host, dev, cap)
    devcache.init_dev_cache(twin, dev, cap)
    w13q = ref.w13_weight.view(torch.uint8).cpu().numpy()
    w2q = ref.w2_weight.view(torch.uint8).cpu().numpy()
    s13 = ref.w13_scale_inv.cpu().numpy()
    s2 = ref.w2_scale_inv.cpu().numpy()
    g = torch.Generator().manual_seed(300 + cap)
    for step, ids_cpu in enumerate(_rows_with_repeats(E, K, 20, cap)):
        ids = ids_cpu.to(dev)
        x = torch.randn((1, H), generator=g).to(torch.bfloat16).to(dev)
        w = torch.softmax(torch.rand((1, K), generator=g), -1).to(dev)
        say(f"devcache fetch_ffn repeats: capacity {cap}, step {step}, ids {ids_cpu.tolist()}")
        monkeypatch.setattr(devcache, "FUSED_FFN", True)
        fused = devcache.dev_cached_forward(host, x, ids, w)
        monkeypatch.setattr(devcache, "FUSED_FFN", False)
        unfused = devcache.dev_cached_forward(twin, x, ids, w)
        want = fp8_moe_forward(x, ids, w, ref.w13_weight, ref.w13_scale_inv, ref.w2_weight,
                               ref.w2_scale_inv)
        torch.cuda.synchronize()
        assert torch.equal(fused, unfused), f"step {step}: fused != unfused"
        assert torch.equal(fused, want), f"step {step}: fused != resident"
        assert torch.equal(host._dc_slot_of, twin._dc_slot_of), f"step {step}"
        assert torch.equal(host._dc_stamp, twin._dc_stamp), f"step {step}"
        if step < 3 or step % 5 == 0:
            oracle_out = omoe.forward_w8a8(x.float().cpu().numpy(), ids_cpu.numpy(),
                                           w.cpu().numpy().astype(np.float64), w13q, s13, w2q, s2)
            err = omoe.max_rel_err(fused.float().cpu().numpy(), oracle_out)
            assert err <= 1e-2, f"step {step}: max rel err {err:.2e} vs the W8A8 oracle"
    hits, misses = devcache.cache_stats(host)
    assert (hits, misses) == devcache.cache_stats(twin)
    assert hits > 0 and misses > 0


@pytest.mark.parametrize("E_,H_,I_,K_,cap", [(24, 8192, 2048, 16, 18), (40, 4096, 1024, 8, 12)],
                         ids=["h8192_i2048_top16", "h4096_i1024"])
def test_hook_fetch_ffn_at_the_limits(lib, dev, E_, H_, I_, K_, cap, monkeypatch):
    """moe_resolve_fetch_ffn at the largest shapes it takes (hidden 8192,
    intermediate 2048, top-16) and at 4096 / 1024: through the hooks, equal
    to the unfused path on a twin cache bit for bit, step for step, with
    equal tables and tile-ordered slot bytes."""
    import devcache
    import moe
    import offload
    import synth
    from hostpool import to_tiles
    monkeypatch.setattr(offload, "DEVICE_TILES", True)
    say(f"devcache fetch_ffn at the limits: E {E_}, H {H_}, I {I_}, top-{K_}, cap {cap}")
    ref = moe.MoEExperts(E_, H_, I_, device=dev)
    synth.fill_experts(ref, seed=8, recipe="devtest", gen_device=dev)
    mods = []
    for _ in range(2):
        m = moe.MoEExperts(E_, H_, I_, device="cpu")
        m._dc_kmax = K_                  # per-call scratch for a top-16 router
        mods.append(m)
    for n in ("w13_weight", "w2_weight", "w13_scale_inv", "w2_scale_inv"):
        pinned = getattr(ref, n).cpu().pin_memory()
        for m in mods:
            setattr(m, n, pinned)
    host, twin = mods
    devcache.init_dev_cache(host, dev, cap)
    devcache.init_dev_cache(twin, dev, cap)
    g = torch.Generator().manual_seed(70 + K_)
    for step in range(12):
        ids = torch.randperm(E_, generator=g)[:K_].view(1, K_).to(dev)
        x = torch.randn((1, H_), generator=g).to(torch.bfloat16).to(dev)
        w = torch.softmax(torch.rand((1, K_), generator=g), -1).to(dev)
        monkeypatch.setattr(devcache, "FUSED_FFN", True)
        fused = devcache.dev_cached_forward(host, x, ids, w)
        monkeypatch.setattr(devcache, "FUSED_FFN", False)
        unfused = devcache.dev_cached_forward(twin, x, ids, w)
        torch.cuda.synchronize()
        assert torch.equal(fused, unfused), f"step {step}"
        assert torch.equal(host._dc_slot_of, twin._dc_slot_of), f"step {step}"
    assert bool(torch.isfinite(fused.float()).all())
    for s_, e in enumerate(host._dc_slot_expert.tolist()):
        if e < 0:
            continue
        assert torch.equal(host._dc_w13[s_].view(torch.uint8).cpu(),
                           to_tiles(host.w13_weight[e].view(torch.uint8))), (s_, e)
        assert torch.equal(host._dc_w2[s_].view(torch.uint8), twin._dc_w2[s_].view(torch.uint8))
    hits, misses = devcache.cache_stats(host)
    assert hits > 0 and misses > 0


def test_capture_dynamic_and_bytes(lib, dev, pair):
    import devcache
    from fp8_moe import fp8_moe_forward
    ref, host = pair
    devcache.init_dev_cache(host, dev, 32)
    ids_warm = torch.randperm(E, device=dev)[:K].unsqueeze(0)
    ids_cap = torch.randperm(E, device=dev)[:K].unsqueeze(0)
    ids_rep = torch.randperm(E, device=dev)[:K].unsqueeze(0)
    ids_live = ids_warm.clone()

    def run():
        return devcache.dev_resolve_and_fetch(host, ids_live)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            run()
    torch.cuda.current_stream().wait_stream(s)
    ids_live.copy_(ids_cap)
    g = torch.cuda.CUDAGraph()
    say("devcache: capture")
    with torch.cuda.graph(g):
        out = run()
    ids_live.copy_(ids_rep)
    g.replay()
    torch.cuda.synchronize()
    slots = out.clone()
    occupant = host._dc_slot_expert[slots.long()]
    assert torch.equal(occupant, ids_rep.reshape(-1).int()), "replay served the wrong experts"
    x = torch.randn(1, H, device=dev).to(torch.bfloat16)
    w = torch.rand(1, K, device=dev)
    w = w / w.sum(-1, keepdim=True)
    want = fp8_moe_forward(x, ids_rep, w, ref.w13_weight, ref.w13_scale_inv, ref.w2_weight,
                           ref.w2_scale_inv)
    got = fp8_moe_forward(x, slots.reshape(1, K), w, host._dc_w13, host._dc_s13, host._dc_w2,
                          host._dc_s2, layout=devcache.cache_layout(host))
    assert torch.equal(want, got)


@pytest.mark.parametrize("coded", [False, True])
def test_whole_decode_layer_graph_replays_match_eager(lib, dev, pair, coded):
    """route -> resolve -> fetch -> experts captured once; several replays,
    eager work and syncs in between, each checked against the same step
    run eagerly on a twin cache (coded: the captured layer fetches from
    coded pools, devcache.CODED_POOL, the eager twin from the raw buffers)."""
    import devcache
    import moe
    import synth
    from fp8_moe import fp8_moe_forward
    ref, host = pair
    host2 = moe.MoEExperts(E, H, I, device="cpu")
    for n in ("w13_weight", "w2_weight", "w13_scale_inv", "w2_scale_inv"):
        setattr(host2, n, getattr(host, n))
    devcache.CODED_POOL = coded
    try:
        devcache.init_dev_cache(host, dev, 24)
    finally:
        devcache.CODED_POOL = False
    devcache.init_dev_cache(host2, dev, 24)
    assert (host._dc_coded is not None) == coded
    gate = synth.router_weight(5, n_experts=E).to(dev)
    x_live = torch.zeros((1, H), dtype=torch.bfloat16, device=dev)
    bias = torch.zeros(E, device=dev)
    rids = torch.empty((1, K), dtype=torch.int64, device=dev)
    rw = torch.empty((1, K), dtype=torch.float32, device=dev)
    rl = torch.empty((1, E), dtype=torch.float32, device=dev)
    out = torch.empty((1, H), dtype=torch.bfloat16, device=dev)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=dev)

    def step(hmod, o):
        moe.route(x_live, gate, K, bias=bias, out=(rids, rw, rl))
        sl = devcache.dev_resolve_and_fetch(hmod, rids)
        fp8_moe_forward(x_live, sl.reshape(1, K), rw, hmod._dc_w13, hmod._dc_s13, hmod._dc_w2,
                        hmod._dc_s2, out=o, workspace=ws, layout=devcache.cache_layout(hmod))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(host, out)
    torch.cuda.current_stream().wait_stream(s)
    devcache.reset_dev_cache(host)                    # fresh table after warm-up
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(host, out)
    devcache.reset_dev_cache(host)
    rng = np.random.default_rng(0)
    twin = torch.empty_like(out)
    for r in range(6):
        x_live.copy_(synth.hidden_states(100 + r, 1).to(dev))
        bias.copy_(torch.from_numpy(rng.gumbel(size=E).astype(np.float32) * 3))
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        _ = torch.randn(1000, device=dev).sum().item()   # eager work between replays
        step(host2, twin)
        torch.cuda.synchronize()
        say(f"graph replay {r}")
        assert torch.equal(got, twin), f"replay {r}"
        assert torch.equal(host._dc_slot_of, host2._dc_slot_of)
        assert torch.equal(host._dc_stamp, host2._dc_stamp)


def test_coded_pool_through_the_hooks_equals_raw(lib, dev, pair):
    """devcache.CODED_POOL: the same decisions, the same cache bytes and the
    same outputs as the raw fetch, step for step."""
    import devcache
    from fp8_moe import fp8_moe_forward
    import moe
    ref, host = pair
    twin = moe.MoEExperts(E, H, I, device="cpu")
    for n in ("w13_weight", "w2_weight", "w13_scale_inv", "w2_scale_inv"):
        setattr(twin, n, getattr(host, n))          # the same pinned tensors
    devcache.init_dev_cache(host, dev, 24)
    devcache.CODED_POOL = True
    try:
        devcache.init_dev_cache(twin, dev, 24)
    finally:
        devcache.CODED_POOL = False
    assert host._dc_coded is None and twin._dc_coded is not None
    say(f"devcache coded pool: ratios {[round(p.ratio, 3) for p in twin._dc_coded]}")
    torch.manual_seed(11)
    for step in range(12):
        x = torch.randn(1, H, device=dev).to(torch.bfloat16)
        ids = torch.randperm(E, device=dev)[:K].unsqueeze(0)
        w = torch.softmax(torch.rand(1, K, device=dev), -1)
        outs = []
        for m in (host, twin):
            slots = devcache.dev_resolve_and_fetch(m, ids)
            outs.append(fp8_moe_forward(x, slots.reshape(ids.shape), w, m._dc_w13, m._dc_s13,
                                        m._dc_w2, m._dc_s2, layout=devcache.cache_layout(m)))
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), f"step {step}"
    for a in ("_dc_w13", "_dc_w2", "_dc_s13", "_dc_s2", "_dc_slot_of", "_dc_stamp"):
        assert torch.equal(getattr(host, a).view(torch.uint8), getattr(twin, a).view(torch.uint8)), a
    assert devcache.cache_stats(host) == devcache.cache_stats(twin)


def test_decode_row_wider_than_the_cache_takes_the_gather(lib, dev, pair):
    """A one-row call with more ids than slots goes to offload's gather
    (the table would give one slot to two ids); the table is not touched
    and the output equals the resident forward's."""
    import devcache
    from fp8_moe import fp8_moe_forward
    ref, host = pair
    devcache.init_dev_cache(host, dev, 4)
    before = [t.clone() for t in (host._dc_slot_of, host._dc_stamp, host._dc_step)]
    x = torch.randn(1, H, device=dev).to(torch.bfloat16)
    ids = torch.randperm(E, device=dev)[:K].unsqueeze(0)
    w = torch.softmax(torch.rand(1, K, device=dev), -1)
    got = devcache.dev_cached_forward(host, x, ids, w)
    want = fp8_moe_forward(x, ids, w, ref.w13_weight, ref.w13_scale_inv, ref.w2_weight,
                           ref.w2_scale_inv)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    for t0, t1 in zip(before, (host._dc_slot_of, host._dc_stamp, host._dc_step)):
        assert torch.equal(t0, t1)


def _twin(host):
    import moe
    t = moe.MoEExperts(E, H, I, device="cpu")
    for n in ("w13_weight", "w2_weight", "w13_scale_inv", "w2_scale_inv"):
        setattr(t, n, getattr(host, n))          # the same pinned tensors
    return t


@pytest.mark.parametrize("cap,ids64", [(9, True), (20, False)])
def test_resolve_fetch_ffn_equals_resolve_then_fetch_ffn(lib, dev, pair, cap, ids64,
                                                         monkeypatch):
    """moe_resolve_fetch_ffn (the resolve made by every workgroup of the
    fetch + gate/up launch, the table staged and copied in by the down
    launch) against moe_resolve_slots followed by moe_fetch_ffn on a twin
    cache, call for call: outputs (bit patterns: an out-of-range id gives a
    NaN row in both), out_slot, the miss list, the counters and the tables
    equal; rows repeat experts and one names an expert past the table."""
    import devcache
    import offload
    ref, host = pair
    twin = _twin(host)
    monkeypatch.setattr(offload, "DEVICE_TILES", True)
    monkeypatch.setattr(devcache, "FUSED_FFN", True)
    devcache.init_dev_cache(host, dev, cap)
    devcache.init_dev_cache(twin, dev, cap)
    lib_ = lib
    rows = _rows_with_repeats(E, K, 24, 40 + cap)
    rows.insert(5, torch.tensor([[1, 2, E + 3, 4, 5, 6, 7, 8]]))
    g = torch.Generator().manual_seed(cap)
    ws = torch.empty(K * I * 4, dtype=torch.uint8, device=dev)
    for step, ids_cpu in enumerate(rows):
        ids = ids_cpu.to(dev) if ids64 else ids_cpu.to(torch.int32).to(dev)
        x = torch.randn((1, H), generator=g).to(torch.bfloat16).to(dev)
        w = torch.softmax(torch.rand((1, K), generator=g), -1).to(dev)
        say(f"resolve_fetch_ffn: capacity {cap}, step {step}, ids {ids_cpu.tolist()}")
        got = devcache.dev_cached_forward(host, x, ids, w)
        # the three-launch form on the twin
        lib_.resolve_slots(ids.reshape(-1), twin._dc_slot_of, twin._dc_slot_expert,
                           twin._dc_stamp, twin._dc_step, twin._dc_out, twin._dc_fslot,
                           twin._dc_fexp, twin._dc_nmiss, twin._dc_stats)
        want = torch.empty_like(x)
        lib_.fetch_ffn(devcache._fetch_pairs(twin, lib_), twin._dc_fexp, twin._dc_fslot,
                       twin._dc_nmiss, K, devcache.CPP_BLOCKS_PER_JOB, x, twin._dc_out[:K],
                       w.reshape(-1), twin._dc_w13, twin._dc_s13, twin._dc_w2, twin._dc_s2,
                       want, ws)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"step {step}"
        n = int(host._dc_nmiss[0])
        assert n == int(twin._dc_nmiss[0]), f"step {step}"
        assert torch.equal(host._dc_out[:K], twin._dc_out[:K]), f"step {step}"
        assert torch.equal(host._dc_fslot[:n], twin._dc_fslot[:n]), f"step {step}"
        assert torch.equal(host._dc_fexp[:n], twin._dc_fexp[:n]), f"step {step}"
        for a in ("_dc_slot_of", "_dc_slot_expert", "_dc_stamp", "_dc_step", "_dc_stats"):
            assert torch.equal(getattr(host, a), getattr(twin, a)), (step, a)
        if step == 5:
            assert bool(torch.isnan(got.float()).all())
    for c_ in ("_dc_w13", "_dc_w2", "_dc_s13", "_dc_s2"):
        assert torch.equal(getattr(host, c_).view(torch.uint8), getattr(twin, c_).view(torch.uint8))


def test_resolve_fetch_ffn_graph_replays_match_eager(lib, dev, pair, monkeypatch):
    """dev_cached_forward on the two-launch path captured once: every replay
    (new ids, new x, eager work and syncs between replays) equals the same
    call made eagerly on a twin cache, tables included."""
    import devcache
    import offload
    ref, host = pair
    twin = _twin(host)
    monkeypatch.setattr(offload, "DEVICE_TILES", True)
    monkeypatch.setattr(devcache, "FUSED_FFN", True)
    devcache.init_dev_cache(host, dev, 16)
    devcache.init_dev_cache(twin, dev, 16)
    ids_live = torch.zeros((1, K), dtype=torch.int64, device=dev)
    x_live = torch.zeros((1, H), dtype=torch.bfloat16, device=dev)
    w_live = torch.full((1, K), 1.0 / K, device=dev)
    rows = _rows_with_repeats(E, K, 8, 77)
    ids_live.copy_(rows[0])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        devcache.dev_cached_forward(host, x_live, ids_live, w_live)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    devcache.reset_dev_cache(host)
    g_ = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_):
        out = devcache.dev_cached_forward(host, x_live, ids_live, w_live)
    devcache.reset_dev_cache(host)
    gen = torch.Generator().manual_seed(3)
    for r, ids_cpu in enumerate(rows):
        x = torch.randn((1, H), generator=gen).to(torch.bfloat16).to(dev)
        ids_live.copy_(ids_cpu)
        x_live.copy_(x)
        g_.replay()
        torch.cuda.synchronize()
        got = out.clone()
        _ = torch.randn(1000, device=dev).sum().item()      # eager work between replays
        want = devcache.dev_cached_forward(twin, x, ids_cpu.to(dev), w_live)
        torch.cuda.synchronize()
        say(f"resolve_fetch_ffn graph replay {r}")
        assert torch.equal(got, want), f"replay {r}"
        for a in ("_dc_slot_of", "_dc_slot_expert", "_dc_stamp", "_dc_step", "_dc_stats"):
            assert torch.equal(getattr(host, a), getattr(twin, a)), (r, a)
