"""The offload dispatch hooks on the GPU (bin/offload.py:137-451; the
reference's bin/test_cache.py checks the same: every path against the
all-resident kernel on the same inputs, exactly).

  * direct (page-locked and pageable host buffers), gather, and the
    host-managed cache give outputs identical to the resident forward, at
    decode- and prefill-shaped calls, with the device rows in MFMA tile
    order (offload.DEVICE_TILES, the default) and row-major;
  * the host-managed cache holds, after every call, exactly the experts its
    decisions put in each slot, in the cache's order (the decisions
    themselves are checked against the oracle on the CPU,
    tests/test_offload_host.py);
  * the direct gather borrows resident experts from the device cache without
    touching its table, counts on the device, and runs without a host sync:
    it is captured in a graph and replayed with new ids.
"""
import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu
E, H, I, K = 32, 2048, 512, 8
_BUFS = ("w13_weight", "w2_weight", "w13_scale_inv", "w2_scale_inv")


@pytest.fixture(scope="module")
def models(dev):
    import moe
    import synth
    ref = moe.MoEExperts(E, H, I, device=dev)
    synth.fill_experts(ref, seed=2, recipe="blockq")
    host = moe.MoEExperts(E, H, I, device="cpu")
    for n in _BUFS:
        host._buffers[n] = getattr(ref, n).cpu().pin_memory()
    host._layer_index = 0
    pageable = moe.MoEExperts(E, H, I, device="cpu")
    for n in _BUFS:
        pageable._buffers[n] = getattr(ref, n).cpu()
    pageable._layer_index = 1
    return ref, host, pageable


def _call(ref, tokens, seed, dev):
    import moe
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn((tokens, H), generator=g).to(torch.bfloat16).to(dev)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(tokens)]).to(dev)
    w = torch.rand((tokens, K), generator=g).to(dev)
    w = w / w.sum(-1, keepdim=True)
    want = moe.MoEExperts._stock_forward(ref, x, ids, w)
    return x, ids, w, want


def _order(tiles):
    from hostpool import to_tiles
    return to_tiles if tiles else (lambda t: t)


@pytest.mark.parametrize("tiles", [True, False])
@pytest.mark.parametrize("mode,which", [("direct", "pinned"), ("direct", "pageable"),
                                        ("gather", "pinned"), ("gather", "pageable")])
def test_copy_modes_match_resident(lib, dev, models, mode, which, tiles, monkeypatch):
    import offload
    ref, host, pageable = models
    layer = host if which == "pinned" else pageable
    monkeypatch.setattr(offload, "DEVICE_TILES", tiles)
    offload.COPY_MODE = mode
    try:
        for step, tokens in enumerate([1, 5, 1, 17, 64]):
            x, ids, w, want = _call(ref, tokens, step, dev)
            say(f"offload: {mode} {which} tiles={tiles} tokens={tokens}")
            before = offload.STATS["experts_copied"]
            got = offload.offloaded_forward(layer, x, ids, w)
            assert torch.equal(got, want)
            n = len(torch.unique(ids))
            assert offload.STATS["experts_copied"] - before == n
    finally:
        offload.COPY_MODE = "direct"


@pytest.mark.parametrize("tiles", [True, False])
def test_hybrid_gather_borrows_device_cache(lib, dev, models, tiles, monkeypatch):
    import devcache
    import offload
    ref, host, _ = models
    monkeypatch.setattr(offload, "DEVICE_TILES", tiles)
    devcache.init_dev_cache(host, dev, 16)
    # the gather rows follow the cache's order whatever the knob says later
    monkeypatch.setattr(offload, "DEVICE_TILES", not tiles)
    try:
        for step in range(6):                      # populate the device cache
            _, ids, _, _ = _call(ref, 1, 50 + step, dev)
            devcache.dev_resolve_and_fetch(host, ids)
        for mode in ("direct", "gather"):
            offload.COPY_MODE = mode
            before = offload.STATS.copy()
            table = [t.clone() for t in (host._dc_slot_of, host._dc_slot_expert, host._dc_stamp,
                                         host._dc_step)]
            x, ids, w, want = _call(ref, 9, 99, dev)
            say(f"offload: hybrid {mode} tiles={tiles}")
            got = offload.offloaded_forward(host, x, ids, w)
            assert torch.equal(got, want)
            resident = set(host._dc_slot_expert.tolist()) - {-1}
            uniq = set(torch.unique(ids).tolist())
            after = offload.STATS.copy()
            assert after["gather_hits"] - before["gather_hits"] == len(uniq & resident)
            assert after["gather_misses"] - before["gather_misses"] == len(uniq - resident)
            for t, u in zip(table, (host._dc_slot_of, host._dc_slot_expert, host._dc_stamp,
                                    host._dc_step)):
                assert torch.equal(t, u)           # read-only use of the table
    finally:
        offload.COPY_MODE = "direct"
        for a in [a for a in vars(host) if a.startswith("_dc_")]:
            delattr(host, a)


def test_direct_gather_is_capturable_and_dynamic(lib, dev, models):
    """No host sync in the direct path: capture one call, replay it with the
    ids (and inputs) of other calls, each replay equal to the resident
    forward on those inputs."""
    import offload
    ref, host, _ = models
    T = 12
    x, ids, w, _ = _call(ref, T, 300, dev)
    offload.offloaded_forward(host, x, ids, w)            # warm-up allocates the gather rows
    xs, idb, wb = x.clone(), ids.clone(), w.clone()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        offload.offloaded_forward(host, xs, idb, wb)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    say("offload: capturing the direct gather")
    with torch.cuda.graph(g):
        out = offload.offloaded_forward(host, xs, idb, wb)
    for r in range(4):
        x, ids, w, want = _call(ref, T, 400 + r, dev)
        xs.copy_(x)
        idb.copy_(ids)
        wb.copy_(w)
        g.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(out, want), f"replay {r}"


def test_captured_gather_survives_a_larger_call(lib, dev, models):
    """A call with more tokens than the shared gather scratch holds grows
    it; a graph captured before still replays correctly, because the old
    scratch is kept (offload._DeviceGather) and the gather rows are shared."""
    import offload
    ref, host, _ = models
    T = 12
    x, ids, w, _ = _call(ref, T, 500, dev)
    offload.offloaded_forward(host, x, ids, w)
    xs, idb, wb = x.clone(), ids.clone(), w.clone()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        offload.offloaded_forward(host, xs, idb, wb)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = offload.offloaded_forward(host, xs, idb, wb)
    retired = len(offload._DeviceGather._retired)
    big = max(g_.max_tokens for g_ in offload._DeviceGather._by_key.values()) + 1
    say(f"offload: a {big}-token call grows the gather scratch")
    xb, ib, wb2, want_b = _call(ref, big, 501, dev)
    got_b = offload.offloaded_forward(host, xb, ib, wb2)
    torch.cuda.synchronize(dev)
    assert torch.equal(got_b, want_b)
    assert len(offload._DeviceGather._retired) == retired + 1
    for r in range(3):
        x, ids, w, want = _call(ref, T, 510 + r, dev)
        xs.copy_(x)
        idb.copy_(ids)
        wb.copy_(w)
        g.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(out, want), f"replay {r} after the scratch grew"
    del g
    torch.cuda.synchronize(dev)
    offload._DeviceGather.release()


@pytest.mark.parametrize("tiles", [True, False])
def test_host_lru_and_fallbacks(lib, dev, models, tiles, monkeypatch):
    import offload
    ref, host, _ = models
    monkeypatch.setattr(offload, "DEVICE_TILES", tiles)
    order = _order(tiles)
    for cap in (8, 12, E):
        offload._init_cache(host, dev, cap)
        say(f"offload: host LRU cap {cap} tiles={tiles}")
        for step in range(12):
            tokens = 1 if step % 3 else 5
            x, ids, w, want = _call(ref, tokens, 1000 + step, dev)
            got = offload.offloaded_forward(host, x, ids, w)
            assert torch.equal(got, want), f"cap {cap} step {step}"
            # every occupied slot holds the expert the decisions put there
            lru = host._lru_state
            for slot in np.nonzero(lru.slot_expert >= 0)[0].tolist():
                e = int(lru.slot_expert[slot])
                for cache, name in zip((host._cache_w13, host._cache_w2, host._cache_s13,
                                        host._cache_s2), _BUFS):
                    want = getattr(host, name)[e].view(torch.uint8)
                    if name.endswith("weight"):
                        want = order(want)
                    assert torch.equal(cache[slot].cpu().view(torch.uint8), want), \
                        f"cap {cap} step {step}: slot {slot} {name}"
    for a in ("_cap", "_cache_w13", "_cache_w2", "_cache_s13", "_cache_s2", "_lru_state",
              "_cache_tiles"):
        delattr(host, a)


def test_graphstub_and_none_modes_run(lib, dev, models):
    import offload
    ref, host, _ = models
    x, ids, w, _ = _call(ref, 1, 7, dev)
    for mode in ("graphstub", "none"):
        offload.COPY_MODE = mode
        try:
            out = offload.offloaded_forward(host, x, ids, w)
            assert out.shape == (1, H) and torch.isfinite(out.float()).all()
        finally:
            offload.COPY_MODE = "direct"


def test_pin_experts_and_device_census(lib, dev):
    """pin_experts re-homes a layer's pageable buffers in one page-locked,
    device-mapped arena (values kept, the fetch kernel can read it); the
    census counts ids on the device."""
    import types
    import devcache
    import moe
    import offload
    import synth
    ex = moe.MoEExperts(E, H, I, device="cpu")
    synth.fill_experts(ex, seed=5)
    want = [getattr(ex, n).clone() for n in _BUFS]
    layer = types.SimpleNamespace(mlp=types.SimpleNamespace(experts=ex))
    model = types.SimpleNamespace(backbone=types.SimpleNamespace(
        model=types.SimpleNamespace(layers=[layer])))
    gib, _ = offload.pin_experts(model, dev)
    assert gib > 0 and all(getattr(ex, n).is_pinned() for n in _BUFS)
    for n, t in zip(_BUFS, want):
        assert torch.equal(getattr(ex, n).view(torch.uint8), t.view(torch.uint8))
    assert offload.pin_experts(model, dev)[0] == 0            # already page-locked
    devcache.init_dev_cache(ex, dev, 8)
    ids = torch.tensor([[3, 1, 4, 15, 9, 2, 6, 5]], device=dev)
    devcache.dev_resolve_and_fetch(ex, ids)
    torch.cuda.synchronize(dev)
    order = _order(ex._dc_tiles)
    for j, e in enumerate(ids[0].tolist()):
        s = int(ex._dc_out[j].item())
        assert torch.equal(ex._dc_w13[s].cpu().view(torch.uint8), order(want[0][e].view(torch.uint8)))
    offload.enable_census(2, E)
    try:
        ex._layer_index = 1
        offload._count(1, ids)
        offload._count(1, ids.repeat(3, 1))
        c = offload.CENSUS[1]
        assert c[3] == 4 and c[0] == 0 and offload.CENSUS_DECODE[1][3] == 1
    finally:
        offload.disable_census()


def test_freed_arena_leaves_no_cached_answers(lib, dev):
    """The device address and the page-locked answer remembered for an
    arena's buffers are dropped when the arena is freed, so an address the
    allocator hands out again is asked afresh."""
    import gc
    import types
    import devcache
    import moe
    import offload
    ex = moe.MoEExperts(8, 256, 128, device="cpu")
    layer = types.SimpleNamespace(mlp=types.SimpleNamespace(experts=ex))
    model = types.SimpleNamespace(backbone=types.SimpleNamespace(
        model=types.SimpleNamespace(layers=[layer])))
    offload.pin_experts(model, dev)
    bufs = [getattr(ex, n) for n in _BUFS]
    addrs = [b.data_ptr() for b in bufs]
    devcache._device_ptr(lib, bufs[0])
    assert offload._all_pinned(bufs)
    assert addrs[0] in devcache._dev_ptr_cache and tuple(addrs) in offload._pinned_memo
    del bufs, layer, model
    del ex
    gc.collect()
    assert addrs[0] not in devcache._dev_ptr_cache
    assert tuple(addrs) not in offload._pinned_memo
