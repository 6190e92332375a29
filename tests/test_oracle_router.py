"""Pin the oracle router: closed-form logits, tie-break, renormalisation."""
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
    lg = router.logits(x, w)
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
    ids, wts, lg = router.route(x, w, 8)
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
    assert np.array_equal(router.logits(x, w), want.float().numpy())
