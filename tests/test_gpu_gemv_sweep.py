"""A seeded sweep of decode-GEMV shapes: hidden 128..4096 (odd K-block
counts included, so the gate/up K halves are unequal), inter 128..1024,
top_k 1..16 (odd ones leave the down kernel's last wave one expert),
1..3 tokens, repeated and out-of-range ids.  Each case: the GEMV output
equals the grouped path's bit for bit, the rows with a bad id are NaN and
the rest are within the oracle bar."""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import moe as omoe

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _cases(n=24, seed=2024):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        H = 128 * int(rng.integers(1, 33))
        I = 128 * int(rng.integers(1, 9))
        K = int(rng.integers(1, 17))
        T = int(rng.integers(1, 4))
        out.append((i, H, I, K, T))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"{c[0]}-H{c[1]}-I{c[2]}-K{c[3]}-T{c[4]}")
def test_gemv_sweep(lib, dev, case):
    import synth
    i, H, I, K, T = case
    E = max(K, 6)
    rng = np.random.default_rng(1000 + i)
    g = torch.Generator(device="cpu").manual_seed(i)
    w13, s13 = synth.quantize_blocks(torch.randn((E, 2 * I, H), generator=g) * 0.02)
    w2, s2 = synth.quantize_blocks(torch.randn((E, H, I), generator=g) * 0.02)
    x = (torch.randn((T, H), generator=g)).to(torch.bfloat16)
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int64)
    if K >= 2:
        ids[0, 1] = ids[0, 0]                    # a repeated expert in token 0
    bad_row = None
    if T >= 2:
        ids[T - 1, K - 1] = E + 3                # an out-of-range id in the last token
        bad_row = T - 1
    w = torch.rand((T, K), generator=g)
    w = w / w.sum(-1, keepdim=True)
    d = [t.to(dev) for t in (w13, s13, w2, s2)]
    xd, idd, wd = x.to(dev), torch.from_numpy(ids).to(dev), w.to(dev)
    ws = torch.empty(lib.fp8_moe_workspace(T, K, E, H, I), dtype=torch.uint8, device=dev)
    a, b = torch.empty_like(xd), torch.empty_like(xd)
    say(f"sweep {i}: H={H} I={I} K={K} T={T}")
    lib.fp8_moe_forward(xd, idd, wd, d[0].view(torch.float8_e4m3fn), d[1],
                        d[2].view(torch.float8_e4m3fn), d[3], a, ws, mode=1)
    lib.fp8_moe_forward(xd, idd, wd, d[0].view(torch.float8_e4m3fn), d[1],
                        d[2].view(torch.float8_e4m3fn), d[3], b, ws, mode=2)
    torch.cuda.synchronize()
    af, bf = a.float().cpu(), b.float().cpu()
    good = [t for t in range(T) if t != bad_row]
    assert torch.equal(af[good], bf[good])
    if bad_row is not None:
        assert torch.isnan(af[bad_row]).all() and torch.isnan(bf[bad_row]).all()
    want = omoe.forward_w8a8(x[good].float().numpy(), ids[good], w[good].numpy().astype(np.float64),
                             w13.numpy(), s13.numpy(), w2.numpy(), s2.numpy())
    assert omoe.max_rel_err(af[good].numpy(), want) <= TOL
