"""moe_linear_bf16, the decode benchmark's non-expert stand-in (y = x W^T,
bf16, 1-4 tokens on the vector units, 5-128 on the matrix cores): against
the float64 product of the same bf16 operands rounded once to bf16 (the f32 sum may round differently on a value close to
a bf16 midpoint: at most 1 ulp, on few outputs; on the matrix cores, an
output whose products cancel may also differ by up to 2^-16 of their
magnitudes' sum), identical for 1, 2 and 4
rows per wave (each row's sum does not depend on the grid), and within 1
ulp of torch's own bf16 matrix-vector product; with an addend, bit-equal to
a torch bf16 add followed by the product."""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import router as orouter

pytestmark = pytest.mark.gpu


def _ulps(a, b):
    """Distance in bf16 steps between two bf16 tensors of finite values."""
    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    # order-preserving map of the sign-magnitude bit patterns
    ka = torch.where(ia < 0, -(ia & 0x7fff), ia)
    kb = torch.where(ib < 0, -(ib & 0x7fff), ib)
    return (ka - kb).abs()


@pytest.mark.parametrize("T,K,N", [(1, 2048, 2048), (3, 2048, 2048), (4, 264, 1001),
                                   (1, 8, 5), (2, 520, 64),
                                   # the matrix-core kernel: 5 to 128 tokens
                                   (5, 2048, 2048), (8, 2048, 2048), (16, 2048, 2048),
                                   (17, 2048, 2048), (32, 2048, 2048), (128, 2048, 2048),
                                   (100, 320, 48), (7, 64, 16), (33, 2112, 80)])
def test_linear_bf16_against_float64(lib, dev, T, K, N):
    g = torch.Generator(device="cpu").manual_seed(K + N + T)
    x = torch.randn((T, K), generator=g).to(torch.bfloat16)
    w = (torch.randn((N, K), generator=g) / K ** 0.5).to(torch.bfloat16)
    exact = x.double() @ w.double().T
    want = torch.from_numpy(orouter.bf16_round(exact.numpy())).to(torch.bfloat16)
    xd, wd = x.to(dev), w.to(dev)
    outs = []
    for rpw in (0, 1, 2, 4):
        y = torch.full((T, N), float("nan"), dtype=torch.bfloat16, device=dev)
        say(f"linear_bf16: T={T} K={K} N={N} rows_per_wave={rpw}")
        lib.linear_bf16(xd, wd, y, rows_per_wave=rpw)
        outs.append(y)
    torch.cuda.synchronize()
    for y in outs[1:]:
        assert torch.equal(y.view(torch.int16), outs[0].view(torch.int16))
    got = outs[0].cpu()
    assert bool(torch.isfinite(got.float()).all())
    d = _ulps(got, want)
    if T <= 4:
        assert int(d.max()) <= 1
    else:
        # the matrix cores' float32 sums: within 1 ulp, or, where the row's
        # products cancel, within 2^-16 of the sum of their magnitudes
        mag = x.double().abs() @ w.double().abs().T
        err = (got.double() - exact).abs()
        assert bool(((d <= 1) | (err <= 2.0 ** -16 * mag)).all())
    assert float((d == 0).float().mean()) >= 0.99
    if T == 1:
        ref = torch.mv(wd, xd[0]).cpu()
        assert int(_ulps(got[0], ref).max()) <= 1


@pytest.mark.parametrize("T,K,N", [(1, 2048, 2048), (4, 264, 1001), (2, 8, 3)])
def test_linear_bf16_with_addend_equals_torch_add_then_product(lib, dev, T, K, N):
    """With x_add the kernel multiplies bf16(x + x_add): bit-equal to a
    torch bf16 add followed by the plain kernel, for every rows_per_wave,
    and the device's bf16 add itself equal to the CPU's."""
    g = torch.Generator(device="cpu").manual_seed(7 * K + N + T)
    x = torch.randn((T, K), generator=g).to(torch.bfloat16)
    r = (torch.randn((T, K), generator=g) * 3).to(torch.bfloat16)
    w = (torch.randn((N, K), generator=g) / K ** 0.5).to(torch.bfloat16)
    xd, rd, wd = x.to(dev), r.to(dev), w.to(dev)
    s = xd + rd
    assert torch.equal(s.cpu().view(torch.int16), (x + r).view(torch.int16))
    plain = torch.empty((T, N), dtype=torch.bfloat16, device=dev)
    lib.linear_bf16(s, wd, plain)
    for rpw in (0, 2, 4):
        y = torch.full((T, N), float("nan"), dtype=torch.bfloat16, device=dev)
        say(f"linear_bf16 x_add: T={T} K={K} N={N} rows_per_wave={rpw}")
        lib.linear_bf16(xd, wd, y, rows_per_wave=rpw, x_add=rd)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), plain.view(torch.int16)), rpw


def test_linear_bf16_preconditions(lib, dev):
    import hipfetch
    x = torch.zeros((129, 64), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((16, 64), dtype=torch.bfloat16, device=dev)
    y = torch.zeros((129, 16), dtype=torch.bfloat16, device=dev)
    with pytest.raises(hipfetch.NativeError, match="tokens"):
        lib.linear_bf16(x, w, y)
    # beyond 4 tokens: K a multiple of 64, N of 16, no addend
    with pytest.raises(hipfetch.NativeError, match="multiple of 64"):
        lib.linear_bf16(x[:5, :56].contiguous(), w[:, :56].contiguous(), y[:5])
    with pytest.raises(hipfetch.NativeError, match="multiple of 64"):
        lib.linear_bf16(x[:5], w[:8], torch.zeros((5, 8), dtype=torch.bfloat16, device=dev))
    with pytest.raises(hipfetch.NativeError, match="x_add NULL"):
        lib.linear_bf16(x[:5], w, y[:5], x_add=x[:5])
    with pytest.raises(hipfetch.NativeError, match="rows_per_wave"):
        lib.linear_bf16(x[:1], w, y[:1], rows_per_wave=3)
    with pytest.raises(ValueError, match="agree"):
        lib.linear_bf16(x[:1, :32], w, y[:1])
    with pytest.raises(ValueError, match="x_add must be bfloat16"):
        lib.linear_bf16(x[:1], w, y[:1], x_add=x[:1].float())
    with pytest.raises(ValueError, match="x_add holds"):
        lib.linear_bf16(x[:2], w, y[:2], x_add=x[:1])
