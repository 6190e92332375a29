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
    checked against the oracle on the kernel's own h and routed y."""
    h = _harness(dev)
    try:
        h.stage(0)
        h.x.copy_(h.x0)
        for l in range(h.cfg.layers):
            say(f"moe block layer {l}")
            h.layer(l)
            torch.cuda.synchronize()
            want = shared.shared_expert(_np(h.h), _np(h.sh_wg[l]), _np(h.sh_wu[l]),
                                        _np(h.sh_wd[l]), _np(h.sh_wsg[l]), routed=_np(h.y),
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
