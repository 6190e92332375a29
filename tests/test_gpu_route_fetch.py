"""moe_route_fetch, the decode step's router + resolve + fetch in two
launches, against moe_route_resolve followed by moe_fetch (three launches),
moe_route_fetch_ffn (the same with the expert FFN, three launches)
against those and the FFN's own two, moe_route_fetch_ffn_uncached (its
0 %-hit form) against moe_router_topk + moe_fetch + the FFN, and
moe_route_fetch_coded (the route in the coded fetch's launch) against
moe_route_resolve + moe_fetch_coded,
at Drama-3 shape (256 experts, top-8, H 2048, I 512) and two others (320
experts, top-12, 272 slots; 64 experts, top-4, 5 slots) over 3 layers and
popularity drifts: two harnesses on the same pools, one per path, step for
step, eager and then replayed from their graphs.  Step outputs, router
outputs, slot decisions, miss queues, hit/miss counters, the current slot
tables (the fused path's double buffer read at step & 1) and every occupied
cache slot are equal.  The tests of the full 40-layer step check the fused
path against the oracle; this one pins it to the separate launches."""
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu


def _same(a, b, tag):
    assert torch.equal(a.x, b.x), f"{tag}: step output"
    for name in ("ids", "wts", "out_slot", "stats", "step"):
        ga, gb = getattr(a, name), getattr(b, name)
        if isinstance(ga, list):
            assert all(torch.equal(u, v) for u, v in zip(ga, gb)), f"{tag}: {name}"
        else:
            assert torch.equal(ga, gb), f"{tag}: {name}"
    for l in range(a.cfg.layers):
        n = int(a.nmiss[l])
        assert n == int(b.nmiss[l]), f"{tag} layer {l}: nmiss"
        assert torch.equal(a.fexp[l][:n], b.fexp[l][:n]) and torch.equal(a.fslot[l][:n], b.fslot[l][:n])
    for ta, tb in zip(a._tables(), b._tables()):
        assert all(torch.equal(u, v) for u, v in zip(ta, tb)), f"{tag}: table"
    se = a._tables()[1]
    for l in range(a.cfg.layers):
        occ = (se[l] >= 0).nonzero().flatten()
        assert torch.equal(a.cache[l][occ], b.cache[l][occ]), f"{tag} layer {l}: cache"


@pytest.mark.parametrize("shape", [
    dict(capacity=20),
    # more jobs than the grid's 8 (each workgroup loops over jobs), the
    # 16-per-lane expert and slot registers (E, cap > 256), 2 workgroups per job
    dict(n_experts=320, top_k=12, hidden=512, inter=256, capacity=272, blocks_per_job=2),
    # a cache one slot above top_k: evictions on almost every step, 1 workgroup per job
    dict(n_experts=64, top_k=4, hidden=256, inter=128, capacity=5, blocks_per_job=1),
], ids=["drama3", "wide", "tight"])
def test_route_fetch_equals_route_resolve_then_fetch(lib, dev, shape):
    import decode
    base = dict(layers=3, drift_every=3, schedule_steps=12, **shape)
    fused = decode.DecodeHarness(decode.DecodeConfig(**base, fused_ffn=False), dev)
    plain = decode.DecodeHarness(decode.DecodeConfig(**base, fused_fetch=False), dev,
                                 pools=fused.pools)
    assert fused.fused and not fused.fused_ffn and not plain.fused
    for s in range(7):
        for h in (fused, plain):
            h.stage(s)
            h.step_eager()
        torch.cuda.synchronize(dev)
        say(f"route_fetch {shape}: eager step {s}")
        _same(fused, plain, f"eager {s}")
    hits, misses = fused.hit_rate()
    assert hits > 0 and misses > 0
    for h in (fused, plain):
        h.capture()
    for s in range(9):
        for h in (fused, plain):
            h.replay(1)
        torch.cuda.synchronize(dev)
        say(f"route_fetch: replay {s}")
        _same(fused, plain, f"replay {s}")
    plain.pools = []                     # owned by the fused harness
    fused.close()


@pytest.mark.parametrize("shape", [
    dict(capacity=20),
    dict(n_experts=320, top_k=12, hidden=512, inter=256, capacity=272, ffn_blocks_per_job=2),
    dict(n_experts=64, top_k=4, hidden=512, inter=128, capacity=5, ffn_blocks_per_job=1),
    # the limits: 1024 experts and slots, top-16 (16 jobs over the grid's 8)
    dict(n_experts=1024, top_k=16, hidden=1024, inter=128, capacity=1024, ffn_blocks_per_job=2),
    # the largest hidden and intermediate sizes (the LDS tables at their
    # maximum: 64 K-blocks, 128 units of 16 columns), at top-16
    dict(n_experts=24, top_k=16, hidden=8192, inter=2048, capacity=18, ffn_blocks_per_job=2),
    dict(n_experts=48, top_k=8, hidden=4096, inter=1024, capacity=12),
], ids=["drama3", "wide", "tight", "limits", "h8192_i2048_top16", "h4096_i1024"])
def test_route_fetch_ffn_equals_separate_launches(lib, dev, shape):
    """moe_route_fetch_ffn (three launches: the misses' gate/up inside the
    fetch, the hits' beside it) against moe_route_resolve + moe_fetch +
    moe_fp8_moe_forward_ex (five): outputs, tables and cache bytes equal
    step for step, eager and replayed."""
    import decode
    base = dict(layers=3, drift_every=3, schedule_steps=12, **shape)
    fused = decode.DecodeHarness(decode.DecodeConfig(**base), dev)
    plain = decode.DecodeHarness(decode.DecodeConfig(**base, fused_fetch=False), dev,
                                 pools=fused.pools)
    assert fused.fused_ffn and not plain.fused
    for s in range(7):
        for h in (fused, plain):
            h.stage(s)
            h.step_eager()
        torch.cuda.synchronize(dev)
        say(f"route_fetch_ffn {shape}: eager step {s}")
        _same(fused, plain, f"eager {s}")
    hits, misses = fused.hit_rate()
    assert hits > 0 and misses > 0
    for h in (fused, plain):
        h.capture()
    for s in range(9):
        for h in (fused, plain):
            h.replay(1)
        torch.cuda.synchronize(dev)
        say(f"route_fetch_ffn: replay {s}")
        _same(fused, plain, f"replay {s}")
    plain.pools = []                     # owned by the fused harness
    fused.close()


@pytest.mark.parametrize("shape", [
    dict(capacity=20),
    dict(n_experts=64, top_k=4, hidden=512, inter=128, capacity=5, ffn_blocks_per_job=1,
         shared_inter=256),
], ids=["drama3", "tight"])
def test_route_fetch_ffn_block_equals_separate_launches(lib, dev, shape):
    """The same with the MoE block's gated shared expert: its gate/up rows in
    the fused launch and its down rows in the down launch, against
    moe_route_resolve + moe_fetch + moe_fp8_moe_block_forward."""
    import decode
    base = dict(layers=3, drift_every=3, schedule_steps=12, shared_expert=True, **shape)
    fused = decode.DecodeHarness(decode.DecodeConfig(**base), dev)
    plain = decode.DecodeHarness(decode.DecodeConfig(**base, fused_fetch=False), dev,
                                 pools=fused.pools)
    assert fused.fused_ffn and not plain.fused
    for s in range(5):
        for h in (fused, plain):
            h.stage(s)
            h.step_eager()
        torch.cuda.synchronize(dev)
        say(f"route_fetch_ffn block {shape}: eager step {s}")
        _same(fused, plain, f"eager {s}")
        assert int(fused.finite) == int(plain.finite) == 1
    for h in (fused, plain):
        h.capture()
    for s in range(6):
        for h in (fused, plain):
            h.replay(1)
        torch.cuda.synchronize(dev)
        say(f"route_fetch_ffn block: replay {s}")
        _same(fused, plain, f"replay {s}")
    plain.pools = []                     # owned by the fused harness
    fused.close()


@pytest.mark.parametrize("fused_ffn", [False, True], ids=["route_fetch", "route_fetch_ffn"])
@pytest.mark.parametrize("shape", [
    dict(capacity=20),
    dict(n_experts=320, top_k=12, hidden=512, inter=256, capacity=272, blocks_per_job=2,
         ffn_blocks_per_job=2),
], ids=["drama3", "wide"])
def test_route_fetch_equals_route_resolve_after_a_long_idle(lib, dev, shape, fused_ffn):
    """The fused route keys a miss's victim by the slots' ages (step -
    stamp) in 20 bits and falls back to the 64-bit stamps when an age
    reaches 2^20 - 1: with every layer's step counter advanced by 2^21 +
    2 between two steps, the slots stamped before are that old, later
    steps mix old and new stamps, and the decisions still equal
    moe_route_resolve's step for step."""
    import decode
    base = dict(layers=2, drift_every=2, schedule_steps=12, **shape)
    fused = decode.DecodeHarness(decode.DecodeConfig(**base, fused_ffn=fused_ffn), dev)
    plain = decode.DecodeHarness(decode.DecodeConfig(**base, fused_fetch=False), dev,
                                 pools=fused.pools)
    assert fused.fused and fused.fused_ffn == fused_ffn and not plain.fused
    for s in range(10):
        if s == 4:
            for h in (fused, plain):          # an even jump keeps the buffer parity
                for st in h.step:
                    st += 2 ** 21 + 2
        for h in (fused, plain):
            h.stage(s)
            h.step_eager()
        torch.cuda.synchronize(dev)
        say(f"route_fetch after a long idle {shape} fused_ffn={fused_ffn}: step {s}")
        _same(fused, plain, f"step {s}")
    hits, misses = fused.hit_rate()
    assert hits > 0 and misses > 0
    plain.pools = []                     # owned by the fused harness
    fused.close()


@pytest.mark.parametrize("shape", [
    dict(capacity=20),
    # E, cap > 256 (16-per-lane registers), 12 jobs over 5 workgroups' 20 waves
    dict(n_experts=320, top_k=12, hidden=512, inter=256, capacity=272, coded_workgroups=5),
    # evictions on almost every step; one workgroup decodes every block
    dict(n_experts=64, top_k=4, hidden=256, inter=128, capacity=5, coded_workgroups=1),
], ids=["drama3", "wide", "tight"])
def test_route_fetch_coded_equals_route_resolve_then_fetch_coded(lib, dev, shape):
    """moe_route_fetch_coded (the route in every workgroup of the coded
    fetch's launch) against moe_route_resolve + moe_fetch_coded on the same
    coded pools: outputs, tables and decoded cache bytes equal step for
    step, eager and replayed."""
    import decode
    base = dict(layers=3, drift_every=3, schedule_steps=12, coded_pool=True, **shape)
    fused = decode.DecodeHarness(decode.DecodeConfig(**base), dev)
    plain = decode.DecodeHarness(decode.DecodeConfig(**base, fused_fetch=False), dev,
                                 pools=fused.pools, coded=fused.coded)
    assert fused.fused and not fused.fused_ffn and not plain.fused
    for s in range(7):
        for h in (fused, plain):
            h.stage(s)
            h.step_eager()
        torch.cuda.synchronize(dev)
        say(f"route_fetch_coded {shape}: eager step {s}")
        _same(fused, plain, f"eager {s}")
    hits, misses = fused.hit_rate()
    assert hits > 0 and misses > 0
    for h in (fused, plain):
        h.capture()
    for s in range(9):
        for h in (fused, plain):
            h.replay(1)
        torch.cuda.synchronize(dev)
        say(f"route_fetch_coded: replay {s}")
        _same(fused, plain, f"replay {s}")
    plain.pools, plain.coded = [], None  # owned by the fused harness
    fused.close()


@pytest.mark.parametrize("shape", [
    dict(),
    # 12 jobs over the grid's 8, the 16-per-lane expert registers (E > 256)
    dict(n_experts=320, top_k=12, hidden=512, inter=256, ffn_blocks_per_job=2),
    dict(n_experts=64, top_k=4, hidden=512, inter=128, ffn_blocks_per_job=1),
    # the MoE block: the shared expert's rows beside the fetch
    dict(n_experts=64, top_k=4, hidden=512, inter=128, shared_expert=True, shared_inter=256),
    # the kernels' limits: hidden 8192, intermediate 2048, top-16
    dict(n_experts=24, top_k=16, hidden=8192, inter=2048, ffn_blocks_per_job=2),
], ids=["drama3", "wide", "tight", "block", "h8192_i2048_top16"])
def test_route_fetch_ffn_uncached_equals_separate_launches(lib, dev, shape):
    """moe_route_fetch_ffn_uncached (0 % hit: every pick fetched into slot
    k, three launches) against moe_router_topk + moe_fetch of the ids into
    slots 0..top_k-1 + moe_fp8_moe_forward (block_forward with the shared
    expert): step outputs, router outputs and every cache slot equal step
    for step, eager and replayed; the fused path's miss lists are the ids
    in slots 0..top_k-1 and its counters, when given, count every pick a
    miss."""
    import decode
    base = dict(layers=3, drift_every=3, schedule_steps=12, mode="nocache", **shape)
    fused = decode.DecodeHarness(decode.DecodeConfig(**base), dev)
    plain = decode.DecodeHarness(decode.DecodeConfig(**base, fused_fetch=False), dev,
                                 pools=fused.pools)
    assert fused.fused_uncached and not plain.fused_uncached and not plain.fused
    K = fused.cfg.top_k
    ar = torch.arange(K, dtype=torch.int32, device=dev)

    def same(tag):
        assert torch.equal(fused.x, plain.x), f"{tag}: step output"
        assert torch.equal(fused.ids, plain.ids) and torch.equal(fused.wts, plain.wts), tag
        for l in range(fused.cfg.layers):
            assert torch.equal(fused.cache[l], plain.cache[l]), f"{tag} layer {l}: cache"
            assert torch.equal(fused.out_slot[l].view(-1), ar), f"{tag} layer {l}: out_slot"
            assert torch.equal(fused.fslot[l], ar), f"{tag} layer {l}: fetch_slot"
            assert torch.equal(fused.fexp[l], fused.ids[l].view(-1)), f"{tag} layer {l}: fetch"
            assert int(fused.nmiss[l]) == K, f"{tag} layer {l}: nmiss"
        if fused.cfg.shared_expert:
            assert int(fused.finite) == int(plain.finite) == 1

    for s in range(5):
        for h in (fused, plain):
            h.stage(s)
            h.step_eager()
        torch.cuda.synchronize(dev)
        say(f"route_fetch_ffn_uncached {shape}: eager step {s}")
        same(f"eager {s}")
    for h in (fused, plain):
        h.capture()
    for s in range(6):
        for h in (fused, plain):
            h.replay(1)
        torch.cuda.synchronize(dev)
        say(f"route_fetch_ffn_uncached: replay {s}")
        same(f"replay {s}")
    # the counters, when given: every pick a miss, added to what they hold
    stats = torch.tensor([5, 7], dtype=torch.int64, device=dev)
    cfg = fused.cfg
    lib.route_fetch_ffn_uncached(fused.h, fused.gate[0], fused.bias_live[0], K, fused.logits[0],
                                 fused.ids[0], fused.wts[0], fused.out_slot[0], fused.fslot[0],
                                 fused.fexp[0], fused.nmiss[0], fused.pools[0].dev_ptr,
                                 fused.cache[0], cfg.inter, cfg.ffn_blocks_per_job, fused.y,
                                 fused.ws_block if cfg.shared_expert else fused.ws,
                                 stats=stats,
                                 shared=fused.shared(0) if cfg.shared_expert else None)
    torch.cuda.synchronize(dev)
    assert stats.tolist() == [5, 7 + K]
    plain.pools = []                     # owned by the fused harness
    fused.close()


def test_route_fetch_preconditions(lib, dev):
    import hipfetch
    E, C, K, H = 256, 16, 8, 256
    i32 = dict(dtype=torch.int32, device=dev)
    x = torch.zeros((1, H), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((E, H), dtype=torch.bfloat16, device=dev)
    logits = torch.zeros(E, device=dev)
    ids, out_slot, fs, fe = (torch.zeros(K, **i32) for _ in range(4))
    wts = torch.zeros(K, device=dev)
    nm = torch.zeros(1, **i32)
    step = torch.zeros(1, dtype=torch.int64, device=dev)
    single = (torch.zeros(E, **i32), torch.zeros(C, **i32), torch.zeros(C, dtype=torch.int64, device=dev))
    pair = [(16, 16, 4096)]
    with pytest.raises(ValueError, match="double-buffered"):
        lib.route_fetch(x, w, None, K, logits, ids, wts, *single, step, out_slot, fs, fe, nm, pair, 3)
    so = torch.zeros((2, E), **i32)
    se = torch.zeros((2, 4), **i32)
    st = torch.zeros((2, 4), dtype=torch.int64, device=dev)
    with pytest.raises(hipfetch.NativeError, match="exceeds the cache capacity"):
        lib.route_fetch(x, w, None, K, logits, ids, wts, so, se, st, step, out_slot, fs, fe, nm,
                        pair, 3)
