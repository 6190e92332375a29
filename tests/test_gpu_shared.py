"""Shared expert and finiteness guard on the GPU, through the C ABI, against
the oracle (oracle/shared.py, itself bit-equal to torch's bf16 modules on the
CPU).  The kernels sum in float32 in their own order, so a bf16 rounding can
land one ulp apart: the bar is >= 99 % bit-equal elements and at most 2 ulp
anywhere, for the intermediate act, the sigmoid gate and the block output."""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import shared

pytestmark = pytest.mark.gpu


def _agree(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    # one bf16 ulp of the larger magnitude: 2^(e - 8) for a value m * 2^e, m in [0.5, 1)
    _, e = np.frexp(np.maximum(np.abs(want), np.abs(got)))
    ulp = np.ldexp(1.0, e - 8) + 1e-30
    return float((got == want).mean()), float((np.abs(got - want) / ulp).max())


def _weights(seed, T, H, Is, dev):
    g = torch.Generator().manual_seed(seed)
    bf = lambda *s, std=1.0: (torch.randn(s, generator=g) * std).to(torch.bfloat16).to(dev)
    return dict(x=bf(T, H), wg=bf(Is, H, std=H ** -0.5), wu=bf(Is, H, std=H ** -0.5),
                wd=bf(H, Is, std=Is ** -0.5), wsg=bf(H, std=H ** -0.5), routed=bf(T, H),
                res=bf(T, H))


def _np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("T,H,Is", [(1, 2048, 512), (3, 256, 128), (37, 2048, 512),
                                    (6, 1024, 384), (2, 8192, 2048)])
def test_shared_expert_matches_oracle(lib, dev, T, H, Is):
    p = _weights(T + H + Is, T, H, Is, dev)
    act = torch.empty((T, Is), dtype=torch.bfloat16, device=dev)
    sig = torch.empty(T, dtype=torch.float32, device=dev)
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    plain = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    say(f"shared expert: T={T} H={H} Is={Is}")
    lib.shared_gate_up(p["x"], p["wg"], p["wu"], p["wsg"], act, sig)
    lib.shared_down(act, sig, p["wd"], out, routed=p["routed"], residual=p["res"])
    lib.shared_down(act, sig, p["wd"], plain)
    torch.cuda.synchronize()
    q = {k: _np(v) for k, v in p.items()}
    want_a, want_s = shared.gate_up(q["x"], q["wg"], q["wu"], q["wsg"])
    for name, got, want in (("act", _np(act), want_a), ("sig", sig.cpu().numpy(), want_s)):
        same, ulps = _agree(got, want)
        assert same >= 0.99 and ulps <= 2.0, (name, same, ulps)
    # the second half from the kernel's own act and sig, then end to end
    same, ulps = _agree(_np(out), shared.down(_np(act), sig.cpu().numpy(), q["wd"], q["routed"],
                                              q["res"]))
    assert same >= 0.99 and ulps <= 2.0, ("down", same, ulps)
    same, ulps = _agree(_np(plain), shared.down(_np(act), sig.cpu().numpy(), q["wd"]))
    assert same >= 0.99 and ulps <= 2.0, ("down plain", same, ulps)
    same, ulps = _agree(_np(out), shared.shared_expert(q["x"], q["wg"], q["wu"], q["wd"], q["wsg"],
                                                       q["routed"], q["res"]))
    print(f"T={T} H={H} Is={Is}: block output {same:.4f} bit-equal, max {ulps:.2f} ulp")
    assert same >= 0.99 and ulps <= 2.0


def test_shared_down_in_place(lib, dev):
    """out may alias routed (the decode step writes the block sum over it)."""
    T, H, Is = 2, 512, 256
    p = _weights(5, T, H, Is, dev)
    act = torch.empty((T, Is), dtype=torch.bfloat16, device=dev)
    sig = torch.empty(T, dtype=torch.float32, device=dev)
    lib.shared_gate_up(p["x"], p["wg"], p["wu"], p["wsg"], act, sig)
    sep = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    lib.shared_down(act, sig, p["wd"], sep, routed=p["routed"], residual=p["res"])
    r = p["routed"].clone()
    lib.shared_down(act, sig, p["wd"], r, routed=r, residual=p["res"])
    torch.cuda.synchronize()
    assert torch.equal(r, sep)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [1, 7, 8, 9, 1000, 252288])
def test_all_finite(lib, dev, dtype, n):
    flag = torch.full((1,), -1, dtype=torch.int32, device=dev)
    x = torch.randn(n, device=dev).to(dtype)
    say(f"all_finite: {dtype} n={n}")
    lib.all_finite(x, flag)
    torch.cuda.synchronize()
    assert int(flag) == 1
    for pos in sorted({0, n // 2, n - 1}):
        for bad in (float("inf"), float("-inf"), float("nan")):
            y = x.clone()
            y[pos] = bad
            lib.all_finite(y, flag)
            torch.cuda.synchronize()
            assert int(flag) == 0, (pos, bad)


def test_all_finite_empty_and_graph_replays(lib, dev):
    flag = torch.full((1,), -1, dtype=torch.int32, device=dev)
    lib.all_finite(torch.empty(0, device=dev), flag)
    torch.cuda.synchronize()
    assert int(flag) == 1
    x = torch.randn(4096, device=dev)
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        lib.all_finite(x, flag)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        lib.all_finite(x, flag)
    for i in range(6):
        bad = i % 2 == 1
        x[1234] = float("nan") if bad else 1.0
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert int(flag) == (0 if bad else 1), i
