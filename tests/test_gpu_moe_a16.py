"""fp8_moe_forward mode 3 (bf16 activations) on the GPU against the
dequantise-then-matmul closed form, oracle.moe.forward_w8a16: float64
dequantised weights times the activations, the reference's CPU expert path
(bin/offload.py; the closed form of notes/13-non-ada-gpus.md:43-53).

Tolerance: max |got - want| / max |want| <= 1e-2 (the stated bar is 2e-2,
bin/test_cache.py:51).  Mode 3 rounds SiLU(gate) * up to bf16 before the
down products and the output to bf16; the closed form rounds only the
output.  The same inputs through the e4m3 path (mode 1) sit 4-5e-2 from
the closed form (the activation quantisation), which each case reports.
"""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import moe as omoe

pytestmark = pytest.mark.gpu
TOL = 1e-2
MODE_GEMV, MODE_GEMV_A16 = 1, 3


def _case(seed, E, H, I, T, K, recipe="blockq"):
    import synth
    g = torch.Generator(device="cpu").manual_seed(seed)
    host = [torch.empty((E, 2 * I, H), dtype=torch.uint8),
            torch.empty((E, 2 * I // 128, H // 128), dtype=torch.float32),
            torch.empty((E, H, I), dtype=torch.uint8),
            torch.empty((E, H // 128, I // 128), dtype=torch.float32)]
    for e in range(E):
        for dst, src in zip(host, synth.expert_tensors(seed, 0, e, H, I, recipe)):
            dst[e] = src
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int64)
    w = torch.rand((T, K), generator=g)
    w = w / w.sum(-1, keepdim=True)
    return host, x, ids, w


def _forward(lib, dev, host, x, ids, w, mode, ids_dtype=torch.int64, w_dtype=torch.float32,
             residual=None, layout=None):
    T, H = x.shape
    E, I = host[2].shape[0], host[2].shape[2]
    K = ids.shape[1]
    if layout is None:
        d = [t.to(dev) for t in host]
        bufs = (d[0].view(torch.float8_e4m3fn), d[1], d[2].view(torch.float8_e4m3fn), d[3])
        kw = {}
    else:
        rec = layout.pack(*(t.to(dev) for t in host))
        bufs = layout.views(rec)
        kw = {"layout": layout.code}
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    ws = torch.empty(lib.fp8_moe_workspace(T, K, E, H, I), dtype=torch.uint8, device=dev)
    lib.fp8_moe_forward(x.to(dev), torch.from_numpy(ids).to(dev, ids_dtype), w.to(dev, w_dtype),
                        *bufs, out, ws, mode=mode,
                        residual=None if residual is None else residual.to(dev), **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("case", [
    (0, 24, 2048, 512, 1, 8),      # the decode shape
    (1, 20, 4096, 1024, 3, 16),
    (2, 4, 8192, 2048, 1, 4),      # the kernels' limits
    (3, 6, 640, 384, 4, 3),        # K-blocks not a multiple of the chunk, odd top_k
    (4, 16, 2048, 512, 20, 5),     # more tokens than mode 0 would send to the GEMV
], ids=lambda c: f"E{c[1]}-H{c[2]}-I{c[3]}-T{c[4]}-K{c[5]}")
def test_a16_matches_the_dequantise_path(lib, dev, case):
    seed, E, H, I, T, K = case
    host, x, ids, w = _case(seed, E, H, I, T, K)
    say(f"a16: H={H} I={I} T={T} K={K}")
    got = _forward(lib, dev, host, x, ids, w, MODE_GEMV_A16)
    got8 = _forward(lib, dev, host, x, ids, w, MODE_GEMV)
    args = (x.float().numpy(), ids, w.numpy().astype(np.float64), *(t.numpy() for t in host))
    want = omoe.forward_w8a16(*args)
    err = omoe.max_rel_err(got, want)
    err8 = omoe.max_rel_err(got8, want)
    print(f"H={H} I={I} T={T} K={K}: mode 3 vs the dequantise path {err:.2e} "
          f"(mode 1: {err8:.2e})")
    assert err <= TOL
    assert err < err8


def test_a16_config0_recipe_devtest(lib, dev):
    """The second recipe of the reference's device-cache test (randn * 0.2
    cast to e4m3, scales U(0.05, 0.15), bin/test_devcache.py:33-37)."""
    host, x, ids, w = _case(5, 16, 2048, 512, 2, 8, recipe="devtest")
    got = _forward(lib, dev, host, x, ids, w, MODE_GEMV_A16)
    want = omoe.forward_w8a16(x.float().numpy(), ids, w.numpy().astype(np.float64),
                              *(t.numpy() for t in host))
    assert omoe.max_rel_err(got, want) <= TOL


def test_a16_dtypes_layouts_and_residual(lib, dev):
    """int32 ids and bf16 weights give the int64 / float32 result (bf16
    weights taken exactly); packed tile-order records the dense row-major
    result; the residual is added as a bf16 tensor add; a rerun is bit-equal."""
    from hostpool import RecordLayout
    H, I, E, T, K = 1024, 256, 9, 3, 6
    host, x, ids, w = _case(6, E, H, I, T, K)
    wb = w.to(torch.bfloat16)
    a = _forward(lib, dev, host, x, ids, wb, MODE_GEMV_A16, w_dtype=torch.float32)
    b = _forward(lib, dev, host, x, ids, wb, MODE_GEMV_A16, ids_dtype=torch.int32,
                 w_dtype=torch.bfloat16)
    c = _forward(lib, dev, host, x, ids, wb, MODE_GEMV_A16,
                 layout=RecordLayout(hidden=H, inter=I, tiled=True))
    d = _forward(lib, dev, host, x, ids, wb, MODE_GEMV_A16)
    assert np.array_equal(a, b) and np.array_equal(a, c) and np.array_equal(a, d)
    res = torch.randn((T, H), generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    r = _forward(lib, dev, host, x, ids, wb, MODE_GEMV_A16, residual=res)
    want = (torch.from_numpy(a).to(torch.bfloat16) + res).float().numpy()
    assert np.array_equal(r, want)


def test_a16_bad_id_poisons_only_its_token(lib, dev):
    H, I, E, T, K = 512, 128, 5, 3, 2
    host, x, ids, w = _case(8, E, H, I, T, K)
    ids[1, 1] = E + 2
    got = _forward(lib, dev, host, x, ids, w, MODE_GEMV_A16)
    assert np.isfinite(got[0]).all() and np.isfinite(got[2]).all()
    assert np.isnan(got[1]).all()


def test_a16_graph_replays_and_noalloc_equal_eager(lib, dev):
    """Mode 3 captured in a hipGraph: every replay, with eager work and a
    synchronisation between replays, equals the eager call; the
    allocation-free entry point gives the same bytes."""
    H, I, E, T, K = 2048, 512, 12, 2, 8
    host, x, ids, w = _case(9, E, H, I, T, K)
    d = [t.to(dev) for t in host]
    bufs = (d[0].view(torch.float8_e4m3fn), d[1], d[2].view(torch.float8_e4m3fn), d[3])
    xd, idd, wd = x.to(dev), torch.from_numpy(ids).to(dev), w.to(dev)
    ws = torch.empty(lib.fp8_moe_workspace(T, K, E, H, I), dtype=torch.uint8, device=dev)
    eager = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    lib.fp8_moe_forward(xd, idd, wd, *bufs, eager, ws, mode=MODE_GEMV_A16)
    out = torch.empty_like(eager)
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        lib.fp8_moe_forward(xd, idd, wd, *bufs, out, ws, mode=MODE_GEMV_A16)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        lib.fp8_moe_forward(xd, idd, wd, *bufs, out, ws, mode=MODE_GEMV_A16)
    for r in range(3):
        out.zero_()
        ws.fill_(0xFF)                     # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
    del g
    na = torch.empty_like(eager)
    lib.fp8_moe_forward_noalloc(xd, idd, wd, *bufs, na, mode=MODE_GEMV_A16)
    torch.cuda.synchronize()
    assert torch.equal(na, eager)
