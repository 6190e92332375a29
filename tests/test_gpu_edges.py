"""Edge cases on the GPU: empty calls, the largest supported shapes, repeated
experts within a token, and the largest expert counts of the router and the
permutation, each against the oracle or against the other kernel path."""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import moe as omoe
from oracle import permute as operm
from oracle import router as orouter

pytestmark = pytest.mark.gpu


def test_empty_calls_touch_nothing(lib, dev):
    H, I, K, E = 256, 128, 4, 8
    x = torch.empty((0, H), dtype=torch.bfloat16, device=dev)
    ids = torch.empty((0, K), dtype=torch.int64, device=dev)
    w = torch.empty((0, K), device=dev)
    w13 = torch.zeros((E, 2 * I, H), dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    w2 = torch.zeros((E, H, I), dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    s13 = torch.ones((E, 2 * I // 128, H // 128), device=dev)
    s2 = torch.ones((E, H // 128, I // 128), device=dev)
    out = torch.empty_like(x)
    ws = torch.empty(lib.fp8_moe_workspace(0, K, E, H, I), dtype=torch.uint8, device=dev)
    say("edges: empty calls")
    for mode in (0, 1, 2):
        lib.fp8_moe_forward(x, ids, w, w13, s13, w2, s2, out, ws, mode=mode)
    gate = torch.zeros((E, H), dtype=torch.bfloat16, device=dev)
    lib.router_topk(x, gate, None, K, torch.empty((0, E), device=dev), ids, w)
    counts = torch.full((E,), -7, dtype=torch.int32, device=dev)
    offsets = torch.full((E + 1,), -7, dtype=torch.int32, device=dev)
    e32 = torch.empty((0,), dtype=torch.int32, device=dev)
    lib.permute(ids, E, counts, offsets, e32, e32)
    n_unique = torch.full((1,), -7, dtype=torch.int32, device=dev)
    uniq = torch.full((E,), -7, dtype=torch.int32, device=dev)
    rank_of = torch.full((E,), -7, dtype=torch.int32, device=dev)
    lib.unique_inverse(ids, E, counts, n_unique, uniq, rank_of, e32)
    lib.unpermute(torch.empty((0, H), device=dev), e32, w, out)
    torch.cuda.synchronize()
    assert counts.tolist() == [0] * E and offsets.tolist() == [0] * (E + 1)
    assert int(n_unique) == 0 and rank_of.tolist() == [-1] * E


def test_largest_expert_shapes(lib, dev):
    """hidden 8192, inter 2048, top_k 16 (the kernels' limits), one token:
    GEMV against the oracle (routing weights zero except three pairs, which
    the fused multiply-add combine passes through exactly) and grouped ==
    GEMV bit for bit."""
    import synth
    E, H, I, K = 16, 8192, 2048, 16
    g = torch.Generator(device=dev).manual_seed(8)
    parts = []
    for _ in range(E):
        a, b = synth.quantize_blocks(torch.randn((1, 2 * I, H), generator=g, device=dev) * 0.02)
        c, d = synth.quantize_blocks(torch.randn((1, H, I), generator=g, device=dev) * 0.02)
        parts.append((a, b, c, d))
    w13 = torch.cat([p[0] for p in parts]); s13 = torch.cat([p[1] for p in parts])
    w2 = torch.cat([p[2] for p in parts]); s2 = torch.cat([p[3] for p in parts])
    x = torch.randn((1, H), generator=g, device=dev).to(torch.bfloat16)
    ids = torch.randperm(E, device=dev)[:K].view(1, K)
    w = torch.zeros((1, K), device=dev)
    live = [0, 7, 15]
    w[0, live] = torch.tensor([0.5, 0.3, 0.2], device=dev)
    ws = torch.empty(lib.fp8_moe_workspace(1, K, E, H, I), dtype=torch.uint8, device=dev)
    say("edges: largest shapes, GEMV and grouped")
    a_out, b_out = torch.empty_like(x), torch.empty_like(x)
    lib.fp8_moe_forward(x, ids, w, w13, s13, w2, s2, a_out, ws, mode=1)
    lib.fp8_moe_forward(x, ids, w, w13, s13, w2, s2, b_out, ws, mode=2)
    torch.cuda.synchronize()
    assert torch.equal(a_out, b_out)
    sel = ids[0, live].cpu()
    want = omoe.forward_w8a8(x.float().cpu().numpy(), np.arange(3)[None], w[0, live].cpu().numpy()[None].astype(np.float64),
                             w13[sel].view(torch.uint8).cpu().numpy(), s13[sel].cpu().numpy(),
                             w2[sel].view(torch.uint8).cpu().numpy(), s2[sel].cpu().numpy())
    err = omoe.max_rel_err(a_out.float().cpu().numpy(), want)
    print(f"largest shapes: max rel err vs W8A8 oracle {err:.2e}")
    assert err <= 1e-2


def test_repeated_experts_in_a_token(lib, dev):
    """The kernels accept an expert twice in one token (a router never does):
    grouped == GEMV, and the row equals the row with the weights merged."""
    import synth
    E, H, I, K, T = 6, 2048, 512, 8, 4
    g = torch.Generator(device=dev).manual_seed(2)
    w13, s13 = synth.quantize_blocks(torch.randn((E, 2 * I, H), generator=g, device=dev) * 0.02)
    w2, s2 = synth.quantize_blocks(torch.randn((E, H, I), generator=g, device=dev) * 0.02)
    x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
    ids = torch.tensor([[0, 0, 1, 2, 3, 4, 5, 0], [1, 1, 1, 1, 1, 1, 1, 1],
                        [5, 4, 3, 2, 1, 0, 5, 4], [2, 3, 2, 3, 2, 3, 2, 3]], device=dev)
    w = torch.rand((T, K), generator=torch.Generator().manual_seed(3)).to(dev)
    ws = torch.empty(lib.fp8_moe_workspace(T, K, E, H, I), dtype=torch.uint8, device=dev)
    a_out, b_out = torch.empty_like(x), torch.empty_like(x)
    say("edges: repeated experts")
    lib.fp8_moe_forward(x, ids, w, w13, s13, w2, s2, a_out, ws, mode=1)
    lib.fp8_moe_forward(x, ids, w, w13, s13, w2, s2, b_out, ws, mode=2)
    torch.cuda.synchronize()
    assert torch.equal(a_out, b_out)
    want = omoe.forward_w8a8(x.float().cpu().numpy(), ids.cpu().numpy(),
                             w.cpu().numpy().astype(np.float64), w13.view(torch.uint8).cpu().numpy(),
                             s13.cpu().numpy(), w2.view(torch.uint8).cpu().numpy(), s2.cpu().numpy())
    assert omoe.max_rel_err(a_out.float().cpu().numpy(), want) <= 1e-2


def test_router_largest_expert_count(lib, dev):
    E, H, K, T = 4096, 256, 32, 5
    g = torch.Generator(device=dev).manual_seed(4)
    x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
    gate = (torch.randn((E, H), generator=g, device=dev) * 0.05).to(torch.bfloat16)
    ids = torch.empty((T, K), dtype=torch.int64, device=dev)
    w = torch.empty((T, K), device=dev)
    logits = torch.empty((T, E), device=dev)
    say("edges: router 4096 experts, top-32")
    lib.router_topk(x, gate, None, K, logits, ids, w)
    torch.cuda.synchronize()
    o_ids, o_w, _ = orouter.route(x.float().cpu().numpy(), gate.float().cpu().numpy(), K)
    assert np.array_equal(ids.cpu().numpy(), o_ids)
    assert np.allclose(w.cpu().numpy(), o_w, rtol=1e-5, atol=1e-7)


def test_permute_largest_expert_count(lib, dev):
    E, T, K = 4096, 4096, 4
    rng = np.random.default_rng(6)
    ids_np = rng.integers(0, E, (T, K))
    ids_np[:50] = 17                                   # one crowded expert
    ids = torch.from_numpy(ids_np).to(dev)
    i32 = dict(dtype=torch.int32, device=dev)
    counts, offsets = torch.empty(E, **i32), torch.empty(E + 1, **i32)
    srt, pos = torch.empty(T * K, **i32), torch.empty(T * K, **i32)
    say("edges: permute 4096 experts, 16384 pairs")
    lib.permute(ids, E, counts, offsets, srt, pos)
    n_unique, uniq, rank_of = torch.empty(1, **i32), torch.empty(E, **i32), torch.empty(E, **i32)
    inv = torch.empty(T * K, **i32)
    lib.unique_inverse(ids, E, counts, n_unique, uniq, rank_of, inv)
    torch.cuda.synchronize()
    c, o, sp, pp = operm.permute(ids_np, E)
    assert np.array_equal(counts.cpu().numpy(), c) and np.array_equal(offsets.cpu().numpy(), o)
    assert np.array_equal(srt.cpu().numpy(), sp) and np.array_equal(pos.cpu().numpy(), pp)
    u, iv = operm.unique_inverse(ids_np)
    n = int(n_unique)
    assert n == u.size and np.array_equal(uniq[:n].cpu().numpy(), u)
    assert np.array_equal(inv.cpu().numpy(), iv.reshape(-1))
