"""The full MoE-block decode step: routed experts through the device cache
plus the gated shared expert on a second stream, and the finiteness guard,
eager and captured in one hipGraph."""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import shared

pytestmark = pytest.mark.gpu


def _agree(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    _, e = np.frexp(np.maximum(np.abs(want), np.abs(got)))
    ulp = np.ldexp(1.0, e - 8) + 1e-30
    return float((got == want).mean()), float((np.abs(got - want) / ulp).max())


def _harness(dev, layers=3):
    import decode
    cfg = decode.DecodeConfig(layers=layers, n_experts=32, top_k=4, hidden=512, inter=256,
                              capacity=10, schedule_steps=8, drift_every=4, gate_std=0.02,
                              shared_expert=True, shared_inter=256)
    return decode.DecodeHarness(cfg, dev)


def _np(t):
    return t.float().cpu().numpy()


def test_block_layers_match_oracle(lib, dev):
    """Each layer's x = h + (routed + shared): the shared part and both sums
    checked against the oracle on the kernel's own h and the routed experts'
    output (recomputed from the layer's cache slots)."""
    h = _harness(dev)
    try:
        h.stage(0)
        h.x.copy_(h.x0)
        routed = torch.empty_like(h.y)
        for l in range(h.cfg.layers):
            say(f"moe block layer {l}")
            h.layer(l)
            w13, s13, w2, s2 = h.views[l]
            lib.fp8_moe_forward(h.h, h.out_slot[l], h.wts[l], w13, s13, w2, s2, routed, h.ws,
                                layout=h.layout.code)
            torch.cuda.synchronize()
            want = shared.shared_expert(_np(h.h), _np(h.sh_wg[l]), _np(h.sh_wu[l]),
                                        _np(h.sh_wd[l]), _np(h.sh_wsg[l]), routed=_np(routed),
                                        residual=_np(h.h))
            same, ulps = _agree(_np(h.x), want)
            assert same >= 0.99 and ulps <= 2.0, (l, same, ulps)
    finally:
        h.close()


def test_block_graph_equals_eager_and_guard(lib, dev):
    h = _harness(dev, layers=4)
    try:
        eager = []
        h.restart()
        for s in range(3):
            h.stage(s)
            h.step_eager()
            h.lib.all_finite(h.x, h.finite)
            torch.cuda.synchronize()
            eager.append(h.x.clone())
        h.capture()
        for s in range(3):
            say(f"moe block graph replay {s}")
            h.replay(1)
            torch.cuda.synchronize()
            assert torch.equal(h.x, eager[s]), s
            assert int(h.finite) == 1
        hits, misses = h.hit_rate()
        assert hits + misses == 3 * 4 * h.cfg.top_k
        # a NaN in one shared weight reaches the output and trips the guard
        h.sh_wd[2][5, 7] = float("nan")
        h.replay(1)
        torch.cuda.synchronize()
        assert int(h.finite) == 0
        h.sh_wd[2][5, 7] = 0.0
        h.replay(1)
        torch.cuda.synchronize()
        assert int(h.finite) == 1
    finally:
        h.close()


def _routed_experts(seed, E, H, I, dev):
    import synth
    g = torch.Generator(device="cpu").manual_seed(seed)
    w13, s13 = synth.quantize_blocks(torch.randn((E, 2 * I, H), generator=g) * 0.02)
    w2, s2 = synth.quantize_blocks(torch.randn((E, H, I), generator=g) * 0.02)
    return [t.to(dev) for t in (w13, s13, w2, s2)]


@pytest.mark.parametrize("T,K,mode", [(1, 8, 0), (2, 8, 0), (1, 15, 0), (1, 16, 0), (5, 8, 0),
                                      (3, 8, 1), (1, 8, 2)])
def test_block_forward_equals_composition(lib, dev, T, K, mode):
    """moe_fp8_moe_block_forward (the shared expert carried by the decode
    launches when T <= 2) against the composition of the three
    separate calls, bit for bit, with and without the residual."""
    E, H, I, Is = 24, 2048, 512, 512
    w13, s13, w2, s2 = _routed_experts(T * 31 + K, E, H, I, dev)
    g = torch.Generator(device="cpu").manual_seed(T + K)
    bf = lambda *s, std=1.0: (torch.randn(s, generator=g) * std).to(torch.bfloat16).to(dev)
    sh = (bf(Is, H, std=0.02), bf(Is, H, std=0.02), bf(H, Is, std=0.01), bf(H, std=0.02))
    x, res = bf(T, H), bf(T, H)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32).to(dev)
    w = torch.softmax(torch.randn((T, K), generator=g), -1).to(dev)
    ws = torch.empty(lib.fp8_moe_block_workspace(T, K, E, H, I, Is), dtype=torch.uint8, device=dev)
    say(f"block forward: T={T} K={K} mode={mode}")
    for r in (None, res):
        got = torch.empty_like(x)
        lib.fp8_moe_block_forward(x, ids, w, w13, s13, w2, s2, sh, got, ws, mode=mode, residual=r)
        routed = torch.empty_like(x)
        lib.fp8_moe_forward(x, ids, w, w13, s13, w2, s2, routed, ws, mode=mode)
        act = torch.empty((T, Is), dtype=torch.bfloat16, device=dev)
        sig = torch.empty(T, dtype=torch.float32, device=dev)
        want = torch.empty_like(x)
        lib.shared_gate_up(x, sh[0], sh[1], sh[3], act, sig)
        lib.shared_down(act, sig, sh[2], want, routed=routed, residual=r)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, want), (r is None, int((got != want).sum()))
