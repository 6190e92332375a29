"""Pin the shared-expert oracle against torch's own bf16 modules on the CPU
(F.linear, F.silu, torch.sigmoid and bf16 tensor arithmetic -- the ops the
model's MoE block is built from), against closed forms, and show that the
check rejects plausible mistakes planted in the oracle's formula."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import shared


def _inputs(seed, T, H, Is):
    g = torch.Generator().manual_seed(seed)
    bf = lambda *s, std=1.0: (torch.randn(s, generator=g) * std).to(torch.bfloat16)
    return dict(x=bf(T, H), wg=bf(Is, H, std=H ** -0.5), wu=bf(Is, H, std=H ** -0.5),
                wd=bf(H, Is, std=Is ** -0.5), wsg=bf(1, H, std=H ** -0.5), routed=bf(T, H),
                res=bf(T, H))


def _torch_block(p):
    x = p["x"]
    a = F.silu(F.linear(x, p["wg"])) * F.linear(x, p["wu"])
    sh = torch.sigmoid(F.linear(x, p["wsg"])) * F.linear(a, p["wd"])
    return p["res"] + (p["routed"] + sh)


def _f32(t):
    return t.float().numpy()


def _oracle(p, **over):
    q = {k: _f32(v) for k, v in p.items()}
    q.update(over)
    return shared.shared_expert(q["x"], q["wg"], q["wu"], q["wd"], q["wsg"], q["routed"], q["res"])


def _agree(got, want):
    """(fraction of bit-equal elements, max |diff| in units of the larger value's bf16 ulp)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    # one bf16 ulp of the larger magnitude: 2^(e - 8) for a value m * 2^e, m in [0.5, 1)
    _, e = np.frexp(np.maximum(np.abs(want), np.abs(got)))
    ulp = np.ldexp(1.0, e - 8) + 1e-30
    return float((got == want).mean()), float((np.abs(got - want) / ulp).max())


@pytest.mark.parametrize("T,H,Is", [(1, 2048, 512), (5, 256, 128), (16, 512, 384)])
def test_oracle_matches_torch_bf16_modules(T, H, Is):
    p = _inputs(T * 7 + H, T, H, Is)
    same, ulps = _agree(_oracle(p), _f32(_torch_block(p)))
    print(f"T={T} H={H} Is={Is}: {same:.4f} bit-equal, max {ulps:.2f} ulp")
    assert same >= 0.98 and ulps <= 2.0


def test_planted_mistakes_are_rejected():
    """Each is a plausible slip in the formula; each must fail the bar above."""
    p = _inputs(3, 4, 512, 256)
    want = _f32(_torch_block(p))
    q = {k: _f32(v) for k, v in p.items()}
    act, sig = shared.gate_up(q["x"], q["wg"], q["wu"], q["wsg"])
    wrong = {
        "gate/up swapped": shared.shared_expert(q["x"], q["wu"], q["wg"], q["wd"], q["wsg"],
                                                q["routed"], q["res"]),
        "no sigmoid gate": shared.down(act, np.ones_like(sig), q["wd"], q["routed"], q["res"]),
        "routed dropped": shared.shared_expert(q["x"], q["wg"], q["wu"], q["wd"], q["wsg"], None,
                                               q["res"]),
        "down rows reversed": shared.shared_expert(q["x"], q["wg"], q["wu"], q["wd"][::-1].copy(),
                                                   q["wsg"], q["routed"], q["res"]),
    }
    for name, got in wrong.items():
        same, ulps = _agree(got, want)
        assert not (same >= 0.98 and ulps <= 2.0), name


def test_closed_forms():
    p = _inputs(11, 3, 256, 128)
    q = {k: _f32(v) for k, v in p.items()}
    # a zero gate row: sigmoid(0) = 0.5 exactly, so the shared output is d / 2
    a, s = shared.gate_up(q["x"], q["wg"], q["wu"], np.zeros_like(q["wsg"]))
    assert (s == 0.5).all()
    half = shared.down(a, s, q["wd"])
    full = shared.down(a, np.ones_like(s), q["wd"])
    assert np.array_equal(half * 2, full)
    # zero down weights: the block is the routed output plus the residual
    out = shared.shared_expert(q["x"], q["wg"], q["wu"], np.zeros_like(q["wd"]), q["wsg"],
                               q["routed"], q["res"])
    want = (p["res"] + p["routed"]).float().numpy()
    assert np.array_equal(out, want)


def test_all_finite():
    assert shared.all_finite(np.ones(10, np.float32))
    for bad in (np.inf, -np.inf, np.nan):
        v = np.ones(37, np.float32)
        v[23] = bad
        assert not shared.all_finite(v)
