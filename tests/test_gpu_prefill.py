"""Device-side prefill gather on the GPU: the gather plan against the
oracle, gathered bytes against the host records, hybrid (cache + host) equal
to host-only byte for byte, and the MoE output through the device path equal
to the resident kernel bit for bit."""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import permute as op

pytestmark = pytest.mark.gpu
E, H, I, K = 64, 2048, 512, 8


def test_gather_plan_matches_oracle(lib, dev):
    rng = np.random.default_rng(3)
    for n_uniq, cap in ((37, 20), (64, 64), (5, 0), (64, 1)):
        uniq = np.sort(rng.choice(E, n_uniq, replace=False)).astype(np.int32)
        slot_of = np.full(E, -1, np.int32)
        if cap:
            res = rng.choice(E, min(cap, E), replace=False)
            slot_of[res] = rng.permutation(cap)[:res.size]
        say(f"gather plan: {n_uniq} experts, cap {cap}")
        t = lambda a: torch.from_numpy(a).to(dev)      # noqa: E731
        u = torch.full((E,), -7, dtype=torch.int32, device=dev)
        u[:n_uniq] = t(uniq)
        n = torch.tensor([n_uniq], dtype=torch.int32, device=dev)
        bufs = [torch.full((E,), -9, dtype=torch.int32, device=dev) for _ in range(4)]
        nh = torch.zeros(1, dtype=torch.int32, device=dev)
        nc = torch.zeros(1, dtype=torch.int32, device=dev)
        stats = torch.zeros(2, dtype=torch.int64, device=dev)
        so = t(slot_of) if cap else None
        lib.gather_plan(u, n, so, cap, bufs[0], bufs[1], nh, bufs[2], bufs[3], nc, stats)
        torch.cuda.synchronize()
        he, hd, cs, cd = op.gather_plan(uniq, slot_of if cap else None, cap)
        assert int(nh) == he.size and int(nc) == cs.size
        for got, want in zip(bufs, (he, hd, cs, cd)):
            assert np.array_equal(got[:want.size].cpu().numpy(), want)
        assert stats.tolist() == [cs.size, he.size]
        if cap:
            assert np.array_equal(so.cpu().numpy(), slot_of)     # read only


@pytest.fixture(scope="module")
def layer(dev):
    """E experts in page-locked host buffers (reference layout) and the same
    experts resident on the GPU."""
    import moe
    import synth
    ref = moe.MoEExperts(E, H, I, device=dev)
    synth.fill_experts(ref, seed=5, recipe="devtest")
    host = moe.MoEExperts(E, H, I, device="cpu")
    for n in ("w13_weight", "w2_weight", "w13_scale_inv", "w2_scale_inv"):
        setattr(host, n, getattr(ref, n).cpu().pin_memory())
    host._layer_index = 0
    return ref, host


def _routing(T, seed, dev):
    rng = np.random.default_rng(seed)
    ids = torch.tensor(np.stack([rng.choice(E, K, replace=False) for _ in range(T)]), device=dev)
    w = torch.rand((T, K), generator=torch.Generator().manual_seed(seed)).to(dev)
    return ids, w / w.sum(-1, keepdim=True)


@pytest.mark.parametrize("tiles", [False, True])
def test_device_prefill_equals_resident_and_gathers_exact_bytes(lib, dev, layer, tiles):
    """The gather rows hold the host's bytes (tiles: w13/w2 in MFMA tile
    order, hostpool.to_tiles of the host's row-major matrices) and the FFN
    over them equals the resident forward."""
    import devcache
    from fp8_moe import fp8_moe_forward
    import hipfetch
    from hostpool import to_tiles
    from prefill import DevicePrefill
    ref, host = layer
    T = 55
    x = torch.randn((T, H), device=dev).to(torch.bfloat16)
    ids, w = _routing(T, 1, dev)
    pf = DevicePrefill.for_experts(host, K, 64, dev, tiles=tiles)
    assert pf.layout == (hipfetch.LAYOUT_TILES if tiles else hipfetch.LAYOUT_ROWS)
    src = [devcache._device_ptr(lib, getattr(host, n)) for n in
           ("w13_weight", "w2_weight", "w13_scale_inv", "w2_scale_inv")]
    say(f"prefill: host-only gather, tiles={tiles}")
    got = pf.forward(x, ids, w, src)
    want = fp8_moe_forward(x, ids, w, ref.w13_weight, ref.w13_scale_inv, ref.w2_weight,
                           ref.w2_scale_inv)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    uniq = torch.unique(ids).cpu()
    n = int(pf.n_unique)
    assert n == uniq.numel() and torch.equal(pf.uniq[:n].cpu(), uniq.to(torch.int32))
    order = to_tiles if tiles else (lambda t: t)
    assert torch.equal(pf.gather[0][:n].view(torch.uint8).cpu(),
                       order(host.w13_weight.view(torch.uint8)[uniq]))
    assert torch.equal(pf.gather[1][:n].view(torch.uint8).cpu(),
                       order(host.w2_weight.view(torch.uint8)[uniq]))
    assert torch.equal(pf.gather[3][:n].cpu(), host.w2_scale_inv[uniq])


def test_hybrid_gather_equals_host_gather(lib, dev, layer):
    import devcache
    from prefill import DevicePrefill
    ref, host = layer
    devcache.init_dev_cache(host, dev, 24)
    for s in range(6):                       # populate the cache through decode calls
        devcache.dev_resolve_and_fetch(host, _routing(1, 100 + s, dev)[0])
    torch.cuda.synchronize()
    table_before = (host._dc_slot_of.clone(), host._dc_stamp.clone(), host._dc_step.clone())
    T = 40
    x = torch.randn((T, H), device=dev).to(torch.bfloat16)
    ids, w = _routing(T, 2, dev)
    pairs = devcache._copy_pairs(host)
    src = [devcache._device_ptr(lib, h) for h, _ in pairs]
    # gather rows in the cache's order (rows borrowed from it are copied as bytes)
    a = DevicePrefill.for_experts(host, K, 64, dev, tiles=host._dc_tiles)
    b = DevicePrefill.for_experts(host, K, 64, dev, tiles=host._dc_tiles)
    say("prefill: hybrid vs host-only gather")
    out_a = a.forward(x, ids, w, src)
    out_b = b.forward(x, ids, w, src, cache=(host._dc_slot_of, host._dc_cap,
                                             [c.data_ptr() for _, c in pairs]))
    torch.cuda.synchronize()
    n = int(a.n_unique)
    for ga, gb in zip(a.gather, b.gather):
        assert torch.equal(ga[:n].view(torch.uint8), gb[:n].view(torch.uint8))
    assert torch.equal(out_a, out_b)
    resident = int((host._dc_slot_of[a.uniq[:n].long()] >= 0).sum())
    assert b.copy_stats() == (resident, n - resident) and resident > 0
    for t0, t1 in zip(table_before, (host._dc_slot_of, host._dc_stamp, host._dc_step)):
        assert torch.equal(t0, t1)               # the table is only read


def test_dev_cached_forward_prefill_equals_resident(lib, dev, layer):
    """A multi-token call on a layer with a device cache goes to offload's
    direct gather (device-side, borrowing the cache) in every copy mode's
    default; its output equals the resident forward's, and the cache table
    is only read."""
    import devcache
    import offload
    from fp8_moe import fp8_moe_forward
    ref, host = layer
    devcache.init_dev_cache(host, dev, 16)
    devcache.dev_resolve_and_fetch(host, _routing(1, 7, dev)[0])
    T = 33
    x = torch.randn((T, H), device=dev).to(torch.bfloat16)
    ids, w = _routing(T, 3, dev)
    stamp = host._dc_stamp.clone()
    say("prefill: dev_cached_forward of 33 tokens")
    assert offload.HYBRID_GATHER and offload.COPY_MODE == "direct"
    got = devcache.dev_cached_forward(host, x, ids, w)
    want = fp8_moe_forward(x, ids, w, ref.w13_weight, ref.w13_scale_inv, ref.w2_weight,
                           ref.w2_scale_inv)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(stamp, host._dc_stamp)


def test_device_prefill_is_capturable_and_dynamic(lib, dev, layer):
    """The device prefill has no host synchronisation, so a whole call is
    captured once and replayed with different routing each time; every
    replay equals the eager call on the same ids (hybrid gather included)."""
    import devcache
    from prefill import DevicePrefill
    ref, host = layer
    devcache.init_dev_cache(host, dev, 20)
    for s in range(4):
        devcache.dev_resolve_and_fetch(host, _routing(1, 200 + s, dev)[0])
    T = 24
    x = torch.randn((T, H), device=dev).to(torch.bfloat16)
    ids_live = torch.zeros((T, K), dtype=torch.int64, device=dev)
    w_live = torch.zeros((T, K), device=dev)
    pairs = devcache._copy_pairs(host)
    src = [devcache._device_ptr(lib, h) for h, _ in pairs]
    cache = (host._dc_slot_of, host._dc_cap, [c.data_ptr() for _, c in pairs])
    pf = DevicePrefill.for_experts(host, K, T, dev, tiles=host._dc_tiles)
    out = torch.empty_like(x)

    def body():
        pf.forward(x, ids_live, w_live, src, cache, out=out)

    ids0, w0 = _routing(T, 50, dev)
    ids_live.copy_(ids0)
    w_live.copy_(w0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    say("prefill: capture")
    with torch.cuda.graph(g):
        body()
    eager = DevicePrefill.for_experts(host, K, T, dev, tiles=host._dc_tiles)
    for r in range(4):
        ids_r, w_r = _routing(T, 60 + r, dev)
        ids_live.copy_(ids_r)
        w_live.copy_(w_r)
        g.replay()
        torch.cuda.synchronize()
        want = eager.forward(x, ids_r, w_r, src, cache)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {r}"


def test_prefill_from_coded_pool_equals_raw_pool(lib, dev):
    """The gather decoded from an entropy-coded pool fills the same rows with
    the same bytes as the raw pool's, so the outputs are equal; a coded pool
    refuses a gather of the reference's four buffers."""
    import codec
    import decode
    from hostpool import HostPool, RecordLayout
    from prefill import DevicePrefill
    lay = RecordLayout(H, I)
    pool = HostPool(E, lay)
    decode.fill_pool_on_gpu(pool, 0, 3, dev)
    coded = codec.CodedPool(pool.array, lay, dev)
    try:
        T = 48
        x = torch.randn((T, H), device=dev).to(torch.bfloat16)
        ids, w = _routing(T, 7, dev)
        a = DevicePrefill.for_records(E, K, 64, dev, lay)
        b = DevicePrefill.for_records(E, K, 64, dev, lay)
        say(f"prefill: coded pool (ratio {coded.ratio:.3f}) vs raw pool")
        out_a = a.forward(x, ids, w, [pool.dev_ptr])
        out_b = b.forward(x, ids, w, None, coded=coded)
        torch.cuda.synchronize()
        n = int(a.n_unique)
        assert torch.equal(a.gather[0][:n], b.gather[0][:n])
        assert torch.equal(out_a, out_b)
        import moe
        four = DevicePrefill.for_experts(moe.MoEExperts(E, H, I, device="cpu"), K, 64, dev)
        with pytest.raises(ValueError, match="packed records"):
            four.gather_experts(ids, None, coded=coded)
    finally:
        coded.close()
        pool.close()


def test_prefill_at_full_size_512_tokens_256_experts(lib, dev):
    """The workload's prefill at its real size: 512 tokens, uniform top-8 of
    256 experts, H 2048 / I 512, through DevicePrefill (host-only gather),
    through offload.offloaded_forward (the hook's direct mode) and through
    the hybrid gather with a 50-slot decode cache.  All three equal the
    all-resident forward bit for bit; 6 sampled tokens against the W8A8
    oracle within 1e-2 (bin/offload.py:137-239, 195-224)."""
    import devcache
    import moe
    import offload
    import synth
    from fp8_moe import fp8_moe_forward
    from oracle import moe as omoe
    from prefill import DevicePrefill
    E_, T = 256, 512
    say("prefill full size: 256 experts on the GPU and page-locked on the host")
    ref = moe.MoEExperts(E_, H, I, device=dev)
    synth.fill_experts(ref, seed=13, recipe="devtest", gen_device=dev)
    host = moe.MoEExperts(E_, H, I, device="cpu")
    for n in ("w13_weight", "w2_weight", "w13_scale_inv", "w2_scale_inv"):
        setattr(host, n, getattr(ref, n).cpu().pin_memory())
    host._layer_index = 0
    rng = np.random.default_rng(512)
    ids = torch.tensor(np.stack([rng.choice(E_, K, replace=False) for _ in range(T)]), device=dev)
    w = torch.softmax(torch.randn((T, K), generator=torch.Generator().manual_seed(5)), -1).to(dev)
    x = synth.hidden_states(21, T, H).to(dev)
    want = fp8_moe_forward(x, ids, w, ref.w13_weight, ref.w13_scale_inv, ref.w2_weight,
                           ref.w2_scale_inv)
    src = [devcache._device_ptr(lib, getattr(host, n)) for n in
           ("w13_weight", "w2_weight", "w13_scale_inv", "w2_scale_inv")]
    say("prefill full size: DevicePrefill, host-only gather")
    pf = DevicePrefill.for_experts(host, K, T, dev, tiles=True)
    got = pf.forward(x, ids, w, src)
    torch.cuda.synchronize()
    n = int(pf.n_unique)
    assert n == int(torch.unique(ids).numel()) and n > 240
    assert torch.equal(got, want)
    del pf
    say("prefill full size: offload.offloaded_forward (direct mode)")
    assert offload.COPY_MODE == "direct"
    got_hook = offload.offloaded_forward(host, x, ids, w)
    torch.cuda.synchronize()
    assert torch.equal(got_hook, want)
    say("prefill full size: hybrid gather with a 50-slot cache")
    devcache.init_dev_cache(host, dev, 50)
    for s in range(12):
        devcache.dev_resolve_and_fetch(host, ids[s * 3:s * 3 + 1])
    torch.cuda.synchronize()
    stamp = host._dc_stamp.clone()
    pairs = devcache._copy_pairs(host)
    hy = DevicePrefill.for_experts(host, K, T, dev, tiles=host._dc_tiles)
    got_hy = hy.forward(x, ids, w, src, cache=(host._dc_slot_of, host._dc_cap,
                                               [c.data_ptr() for _, c in pairs]))
    torch.cuda.synchronize()
    from_cache, from_host = hy.copy_stats()
    assert from_cache > 0 and from_cache + from_host == n
    assert torch.equal(got_hy, want)
    assert torch.equal(stamp, host._dc_stamp)
    say("prefill full size: 6 tokens against the W8A8 oracle")
    w13q = ref.w13_weight.view(torch.uint8).cpu().numpy()
    w2q = ref.w2_weight.view(torch.uint8).cpu().numpy()
    s13, s2 = ref.w13_scale_inv.cpu().numpy(), ref.w2_scale_inv.cpu().numpy()
    rows = [0, 97, 200, 311, 450, 511]
    ora = omoe.forward_w8a8(x[rows].float().cpu().numpy(), ids[rows].cpu().numpy(),
                            w[rows].cpu().numpy().astype(np.float64), w13q, s13, w2q, s2)
    err = omoe.max_rel_err(got[rows].float().cpu().numpy(), ora)
    print(f"prefill full size: {n} experts, {from_cache} from the cache; "
          f"max rel err vs the W8A8 oracle on 6 tokens {err:.2e}")
    assert err <= 1e-2
