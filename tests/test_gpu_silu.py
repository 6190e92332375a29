"""The expert kernels' SiLU(gate) * up (common.hpp silu_mul: hardware exp2
and reciprocal) against float64, through moe_silu_check.

Bar: |got - want| <= (2 |g| + 8) * 2^-24 * |want| + the float32 denormal
floor.  The rounded argument -g log2 e alone puts about 0.7 |g| * 2^-24 of
relative error into exp2; the hardware exp2 adds more at large arguments
(the measured worst case is about 1.07 * (|g| + 5) * 2^-24, near
|g| = 22.5).  The e4m3 step the result is quantised to is 2^-3.
Special values follow g / (1 + e^-g) * u: -0 past the exp2 overflow, NaN
in, NaN out, +inf gate gives u * inf."""
import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu


def _silu64(g, u):
    g = g.astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        return g / (1.0 + np.exp(-g)) * u.astype(np.float64)


def test_silu_accuracy_dense_grid(lib, dev):
    rng = np.random.default_rng(0)
    n = 1 << 22
    g = np.concatenate([np.linspace(-40.0, 40.0, n // 2, dtype=np.float32),
                        (rng.standard_normal(n // 2) * 4).astype(np.float32)])
    u = (rng.standard_normal(n) * 2).astype(np.float32)
    say("silu: dense grid")
    out = torch.empty(n, dtype=torch.float32, device=dev)
    lib.silu_check(torch.from_numpy(g).to(dev), torch.from_numpy(u).to(dev), out)
    got = out.cpu().numpy().astype(np.float64)
    want = _silu64(g, u)
    ag = np.abs(g.astype(np.float64))
    bound = (2 * ag + 8) * 2.0 ** -24 * np.abs(want) + 2.0 ** -126
    err = np.abs(got - want)
    ulps = err / (np.abs(want) * 2.0 ** -24 + 2.0 ** -149)
    for lo, hi in ((0, 1), (1, 5), (5, 10), (10, 20), (20, 40)):
        m = (ag >= lo) & (ag < hi) & (np.abs(want) > 2.0 ** -126)
        print(f"silu: |g| in [{lo}, {hi}): worst {float(np.max(ulps[m])):.1f} x 2^-24 relative")
    print(f"silu: worst error / bound = {float(np.max(err / bound)):.3f}")
    assert np.all(err <= bound), int(np.argmax(err - bound))


def test_silu_special_values(lib, dev):
    g = np.array([0.0, -0.0, -100.0, -88.0, 100.0, np.inf, -np.inf, np.nan, 1.0], np.float32)
    u = np.array([1.0, 1.0, 1.0, 2.0, 3.0, 1.0, 1.0, 1.0, np.nan], np.float32)
    out = torch.empty(len(g), dtype=torch.float32, device=dev)
    lib.silu_check(torch.from_numpy(g).to(dev), torch.from_numpy(u).to(dev), out)
    got = out.cpu().numpy()
    assert got[0] == 0.0 and got[1] == 0.0
    assert got[2] == 0.0 and np.signbit(got[2])          # -100 / inf = -0
    assert abs(got[3]) < 1e-35                           # -88: e^-88 scale, tiny
    assert got[4] == 300.0                               # 100 * 1 * 3
    assert got[5] == np.inf
    assert np.isnan(got[6]) or got[6] == 0.0             # -inf * 0: NaN (g / inf is NaN too)
    assert np.isnan(got[7]) and np.isnan(got[8])
