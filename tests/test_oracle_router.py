"""Pin the oracle router: closed-form logits, tie-break, renormalisation,
the bf16 rounding of the logits (exact brute force and torch's own bf16
Linear), and the rate at which the bf16 and float32 logit contracts pick a
different top-8."""
import bisect
from fractions import Fraction

import numpy as np
import torch

from oracle import router


def test_logits_closed_form_and_orientation():
    """W = scaled identity rows: logit[e] = c_e * x[e]; a transposed operand
    or a dropped term gives different numbers."""
    H, E = 64, 16
    x = np.arange(1, H + 1, dtype=np.float32)[None, :] / 8.0
    w = np.zeros((E, H), np.float32)
    for e in range(E):
        w[e, e * 3] = (e + 1) / 4.0
    w[5, 7] = -1.0                                   # second term on one row
    lg = router.logits(x, w, logit_dtype="f32")
    want = np.array([(e + 1) / 4.0 * (e * 3 + 1) / 8.0 for e in range(E)], np.float32)
    want[5] += -1.0 * 8 / 8.0
    assert np.array_equal(lg[0], want)


def test_topk_descending_with_low_index_tie_break():
    lg = np.array([[1.0, 3.0, 3.0, 2.0, 3.0, -1.0]], np.float32)
    ids, w = router.topk(lg, 4)
    assert ids.tolist() == [[1, 2, 4, 3]]
    ex = np.exp(np.array([3, 3, 3, 2.0]) - 3)
    np.testing.assert_allclose(w[0], ex / ex.sum(), rtol=1e-15)


def test_renormalised_weights_equal_full_softmax_then_renorm():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 128)).astype(np.float32)
    w = (rng.standard_normal((32, 128)) * 0.5).astype(np.float32)
    ids, wts, lg = router.route(x, w, 8, logit_dtype="f32")
    p = torch.softmax(torch.from_numpy(lg).double(), dim=-1)
    tv, ti = torch.topk(p, 8)
    assert np.array_equal(ti.numpy(), ids)
    np.testing.assert_allclose((tv / tv.sum(-1, keepdim=True)).numpy(), wts, rtol=1e-12)
    assert np.allclose(wts.sum(-1), 1.0)


def test_logits_equal_float64_matmul_rounded_once():
    rng = np.random.default_rng(1)
    x = torch.from_numpy(rng.standard_normal((3, 2048)).astype(np.float32)).bfloat16().float().numpy()
    w = torch.from_numpy((rng.standard_normal((256, 2048)) * 0.02).astype(np.float32)).bfloat16().float().numpy()
    want = torch.from_numpy(x).double() @ torch.from_numpy(w).double().T
    assert np.array_equal(router.logits(x, w, logit_dtype="f32"), want.float().numpy())


def _all_bf16():
    """Every finite bf16 value, ascending, as Python floats."""
    u = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    v = u.double().numpy()
    keep = np.isfinite(v)
    return sorted(set(float(a) for a in v[keep]))


def _nearest_bf16_exact(d: float, grid) -> float:
    """Brute force: the two grid neighbours of d, compared in exact
    rational arithmetic; a tie goes to the even bf16 bit pattern."""
    i = bisect.bisect_left(grid, d)
    if i < len(grid) and grid[i] == d:
        return d
    lo, hi = grid[i - 1], grid[i]
    dl, dh = Fraction(d) - Fraction(lo), Fraction(hi) - Fraction(d)
    if dl != dh:
        return lo if dl < dh else hi
    bits = lambda v: int(torch.tensor([v], dtype=torch.float32).view(torch.int32)) >> 16
    return lo if bits(lo) % 2 == 0 else hi


def test_bf16_round_exact_against_brute_force():
    grid = _all_bf16()
    rng = np.random.default_rng(7)
    vals = list(rng.standard_normal(3000) * np.exp2(rng.integers(-20, 20, 3000)))
    # midpoints of neighbouring bf16 values and the doubles right beside them
    picks = rng.integers(1, len(grid) - 1, 400)
    for i in picks:
        a, b = grid[i], grid[i + 1]
        if not (np.isfinite(a) and np.isfinite(b)):
            continue
        m = (a + b) / 2                                 # exact in float64
        vals += [m, np.nextafter(m, -np.inf), np.nextafter(m, np.inf)]
    vals += list(rng.uniform(-1, 1, 200) * 2.0 ** -128)  # bf16 subnormal range
    vals = np.array(vals, np.float64)
    got = router.bf16_round(vals)
    want = np.array([_nearest_bf16_exact(float(v), grid) for v in vals], np.float64)
    assert np.array_equal(got.astype(np.float64), want)
    # rounding to float32 first, then to bf16, double-rounds the doubles just
    # past a midpoint onto the even neighbour; the vectors above include them
    near = np.array([np.nextafter((grid[i] + grid[i + 1]) / 2, np.inf) for i in picks
                     if grid[i] > 0 and np.isfinite(grid[i + 1])])
    twice = torch.from_numpy(near.astype(np.float32)).to(torch.bfloat16).double().numpy()
    assert np.any(twice != router.bf16_round(near).astype(np.float64))


def test_bf16_round_equals_torch_cast_of_float32_values():
    rng = np.random.default_rng(8)
    f = (rng.standard_normal(100_000) * np.exp2(rng.integers(-30, 30, 100_000))).astype(np.float32)
    want = torch.from_numpy(f).to(torch.bfloat16).float().numpy()
    assert np.array_equal(router.bf16_round(f.astype(np.float64)), want)


def test_bf16_logits_equal_torch_bf16_linear():
    """The gate as the model runs it: torch.nn.functional.linear on bf16
    tensors (float32 accumulation, one rounding to bf16).  torch's float32
    sum and the oracle's exact sum round to different bf16 neighbours only
    when they straddle a rounding boundary: rare, and one ulp at most.  The
    float32 contract is a different function (almost no logit is a bf16
    value), which is what this test would catch."""
    rng = np.random.default_rng(9)
    x = torch.from_numpy(rng.standard_normal((64, 2048)).astype(np.float32)).bfloat16()
    w = torch.from_numpy((rng.standard_normal((256, 2048)) * 0.02).astype(np.float32)).bfloat16()
    want = torch.nn.functional.linear(x, w).float().numpy()
    got = router.logits(x.float().numpy(), w.float().numpy())
    equal = np.mean(got == want)
    ulp = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64)) >> 16
    print(f"bf16 logits equal to torch's bf16 F.linear: {equal:.5f}, max {ulp.max()} ulp")
    assert equal >= 0.999 and ulp.max() <= 1
    f32 = router.logits(x.float().numpy(), w.float().numpy(), logit_dtype="f32")
    assert np.mean(f32 == want) < 0.05


def test_bf16_tie_goes_to_the_lower_expert():
    """Logits 1 + 2^-10 (expert 3) and 1 + 2^-11 (expert 1) both round to
    1.0 in bf16: the tie goes to expert 1.  Under float32 logits expert 3
    ranks first."""
    H, E = 8, 6
    x = np.zeros((1, H), np.float32)
    x[0, 0] = 1.0
    x[0, 1] = 2.0 ** -10
    x[0, 2] = 2.0 ** -11
    w = np.zeros((E, H), np.float32)
    w[3, 0], w[3, 1] = 1.0, 1.0
    w[1, 0], w[1, 2] = 1.0, 1.0
    w[5, 0] = 0.5
    ids, _, lg = router.route(x, w, 2)
    assert lg[0, 1] == lg[0, 3] == 1.0 and ids.tolist() == [[1, 3]]
    ids32, _, _ = router.route(x, w, 2, logit_dtype="f32")
    assert ids32.tolist() == [[3, 1]]


def _disagreement(x, w, bias=None, k=8):
    a, _, _ = router.route(x, w, k, bias, "bf16")
    b, _, _ = router.route(x, w, k, bias, "f32")
    return float(np.mean([set(p) != set(q) for p, q in zip(a.tolist(), b.tolist())]))


def test_contract_disagreement_rates():
    """How often the bf16 and float32 logit contracts select a different set
    of 8 experts.  Upstream-like routing (gate N(0, 0.02), hidden N(0, 1),
    no bias): a few percent of tokens.  The decode workload's routing
    (gate N(0, 0.002) plus the per-layer Zipf popularity bias) is dominated
    by the bias: almost never."""
    import synth
    rng = np.random.default_rng(10)
    x = torch.from_numpy(rng.standard_normal((1024, 2048)).astype(np.float32)).bfloat16().float().numpy()
    w = torch.from_numpy((rng.standard_normal((256, 2048)) * 0.02).astype(np.float32)).bfloat16().float().numpy()
    plain = _disagreement(x, w)
    w2 = torch.from_numpy((rng.standard_normal((256, 2048)) * 0.002).astype(np.float32)).bfloat16().float().numpy()
    bias = synth.decode_route_bias(np.random.default_rng(0), 8, 4, 256, 1.1, 4)   # [steps, L, E]
    rates = [_disagreement(x[:256], w2, bias[s, l]) for s in range(2) for l in range(4)]
    print(f"top-8 sets differing between bf16 and f32 logits: upstream-like {plain:.4f}, "
          f"decode workload {np.mean(rates):.4f}")
    assert 0.0 < plain < 0.2
    assert np.mean(rates) < plain
