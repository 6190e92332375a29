"""The decode step through the reference's hooks at Drama-3 shape (256
experts, H 2048, I 512, top-8).

MoEExperts modules hold the reference's four host buffers, filled from the
packed pools (HostPool.to_experts) and page-locked by offload.pin_experts;
devcache.install_dev_cache gives each layer its cache; every layer calls
experts(h, ids, w) (dev_cached_forward: moe_resolve_slots, one four-buffer
moe_fetch writing w13/w2 in tile order, the expert FFN).  Against the
packed-record harness (decode.DecodeHarness) on the same pools, router,
stub and schedule, step for step across popularity drifts, eager and then
replayed from one hipGraph each:
  * the step outputs are equal bit for bit;
  * after every step each layer's slot table (slot_of, slot_expert, stamp,
    step) and hit/miss counters are equal;
  * every occupied slot of the hooks' cache holds the same w13/w2 bytes
    (tile order) and scales as the harness's packed cache slot.
"""
import types

import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu


def _hooked_layers(hc, dev):
    import devcache
    import moe
    import offload
    cfg = hc.cfg
    mods = [moe.MoEExperts(cfg.n_experts, cfg.hidden, cfg.inter, device="cpu")
            for _ in range(cfg.layers)]
    model = types.SimpleNamespace(backbone=types.SimpleNamespace(model=types.SimpleNamespace(
        layers=[types.SimpleNamespace(mlp=types.SimpleNamespace(experts=m)) for m in mods])))
    offload.pin_experts(model, dev)
    for pool, m in zip(hc.pools, mods):
        pool.to_experts(m, dev)
    torch.cuda.synchronize(dev)
    assert devcache.install_dev_cache(model, dev, cfg.capacity) == cfg.layers
    return mods


def _check_tables(hc, mods, tag):
    lay = hc.layout
    for l, m in enumerate(mods):
        assert torch.equal(hc.slot_of[l], m._dc_slot_of), (tag, l)
        assert torch.equal(hc.slot_expert[l], m._dc_slot_expert), (tag, l)
        assert torch.equal(hc.stamp[l], m._dc_stamp), (tag, l)
        assert torch.equal(hc.step[l], m._dc_step), (tag, l)
        assert torch.equal(hc.stats[l], m._dc_stats), (tag, l)
        occupied = (m._dc_slot_expert >= 0).nonzero().flatten()
        rec = hc.cache[l][occupied]
        # fp8 tensors are indexed through their byte views
        assert torch.equal(rec[:, :lay.off_w2], m._dc_w13.view(torch.uint8)[occupied].flatten(1))
        assert torch.equal(rec[:, lay.off_w2:lay.off_s13],
                           m._dc_w2.view(torch.uint8)[occupied].flatten(1))
        assert torch.equal(rec[:, lay.off_s13:lay.off_s2],
                           m._dc_s13[occupied].flatten(1).view(torch.uint8))


def test_hooks_step_equals_packed_step(lib, dev):
    import decode
    import devcache
    import moe
    cfg = decode.DecodeConfig(layers=3, capacity=24, drift_every=3, schedule_steps=12)
    hc = decode.DecodeHarness(cfg, dev)
    stock = moe.MoEExperts.forward
    try:
        mods = _hooked_layers(hc, dev)
        assert all(m._dc_tiles for m in mods)
        L, E, K = cfg.layers, cfg.n_experts, cfg.top_k
        i32 = dict(dtype=torch.int32, device=dev)
        ids = torch.zeros((L, 1, K), **i32)
        wts = torch.zeros((L, 1, K), dtype=torch.float32, device=dev)
        logits = torch.zeros((L, 1, E), dtype=torch.float32, device=dev)
        x = hc.x0.clone()
        h = torch.empty_like(x)

        def hooked_step():
            x.copy_(hc.x0)
            for l in range(L):
                decode.stub_linear(x, hc.w_stub[l], h)
                lib.router_topk(h, hc.gate[l], hc.bias_live[l], K, logits[l], ids[l], wts[l],
                                logit_dtype=cfg.router_logits)
                y = mods[l](h, ids[l], wts[l])
                torch.add(h, y, out=x)

        for s in range(6):                        # eager, two drifts
            hc.stage(s)
            hc.step_eager()
            hooked_step()
            torch.cuda.synchronize(dev)
            say(f"drop-in full shape: eager step {s}")
            assert torch.equal(x, hc.x), f"eager step {s}"
            _check_tables(hc, mods, f"eager {s}")
        assert int(hc.stats[:, 1].sum()) > 0 and int(hc.stats[:, 0].sum()) > 0

        hc.capture()                              # warm-up, capture, tables reset
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            hc.stage(0)
            hooked_step()
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            hooked_step()
        for m in mods:
            devcache.reset_dev_cache(m)
        for s in range(8):
            hc.replay(1)                          # stages step s, replays
            g.replay()
            torch.cuda.synchronize(dev)
            say(f"drop-in full shape: replay {s}")
            assert torch.equal(x, hc.x), f"replay {s}"
            _check_tables(hc, mods, f"replay {s}")
    finally:
        moe.MoEExperts.forward = stock
        devcache._dev_ptr_cache.clear()
