"""fp8_moe_forward on the GPU against the oracle's W8A8 restatement.

Tolerance: max |got - want| / max |want| <= 1e-2 against oracle.moe.forward_w8a8
(the stated bf16/fp8 bar is 2e-2, bin/test_cache.py:51).  The distance to the
dequantise-then-matmul path (oracle.moe.forward_w8a16) is the activation
quantisation error (4.2-4.5 % on these inputs, computed oracle to oracle)
and is reported, bounded at 6e-2.
"""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import moe as omoe

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _experts(seed, E, H, I, recipe, dev):
    import synth
    w13 = torch.empty((E, 2 * I, H), dtype=torch.uint8)
    s13 = torch.empty((E, 2 * I // 128, H // 128), dtype=torch.float32)
    w2 = torch.empty((E, H, I), dtype=torch.uint8)
    s2 = torch.empty((E, H // 128, I // 128), dtype=torch.float32)
    for e in range(E):
        a, b, c, d = synth.expert_tensors(seed, 0, e, H, I, recipe)
        w13[e], s13[e], w2[e], s2[e] = a, b, c, d
    host = (w13, s13, w2, s2)
    devt = tuple(t.to(dev) for t in host)
    return host, devt


def _np(t):
    return t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


def _run(x, ids, w, devt, **kw):
    from fp8_moe import fp8_moe_forward
    w13, s13, w2, s2 = devt
    return fp8_moe_forward(x, ids, w, w13.view(torch.float8_e4m3fn), s13,
                           w2.view(torch.float8_e4m3fn), s2, **kw)


@pytest.mark.parametrize("recipe", ["blockq", "devtest"])
def test_decode_one_token_eight_experts(lib, dev, recipe):
    import synth
    E, H, I = 24, 2048, 512
    host, devt = _experts(0, E, H, I, recipe, dev)
    x = synth.hidden_states(0, 1).to(dev)
    rng = np.random.default_rng(1)
    ids = torch.tensor(rng.choice(E, 8, replace=False)[None, :], dtype=torch.int64, device=dev)
    w = torch.rand((1, 8), generator=torch.Generator().manual_seed(2)).to(dev)
    w = w / w.sum(-1, keepdim=True)
    say(f"moe: decode 1x8 {recipe}")
    got = _run(x, ids, w, devt)
    torch.cuda.synchronize()
    args = (_np(x), ids.cpu().numpy(), w.cpu().numpy().astype(np.float64),
            host[0].numpy(), host[1].numpy(), host[2].numpy(), host[3].numpy())
    want = omoe.forward_w8a8(*args)
    err = omoe.max_rel_err(_np(got), want)
    gap = omoe.max_rel_err(_np(got), omoe.forward_w8a16(*args))
    print(f"{recipe}: max rel err vs W8A8 oracle {err:.2e}, vs W8A16 {gap:.2e}")
    assert err <= TOL
    assert gap <= 6e-2


def test_several_tokens_and_dtypes(lib, dev):
    import synth
    E, H, I, T, K = 12, 2048, 512, 5, 8
    host, devt = _experts(3, E, H, I, "blockq", dev)
    x = synth.hidden_states(3, T).to(dev)
    rng = np.random.default_rng(4)
    ids = torch.tensor(np.stack([rng.choice(E, K, replace=False) for _ in range(T)]),
                       dtype=torch.int32, device=dev)
    w = torch.rand((T, K), generator=torch.Generator().manual_seed(5)).to(dev)
    w = (w / w.sum(-1, keepdim=True)).to(torch.bfloat16)
    say("moe: 5 tokens, int32 ids, bf16 weights")
    got = _run(x, ids, w, devt)
    got64 = _run(x, ids.long(), w.float(), devt)
    torch.cuda.synchronize()
    assert torch.equal(got, got64)           # bf16 weights are exact in f32
    want = omoe.forward_w8a8(_np(x), ids.cpu().numpy(), w.float().cpu().numpy().astype(np.float64),
                             *(t.numpy() for t in host))
    assert omoe.max_rel_err(_np(got), want) <= TOL


def test_small_shapes(lib, dev):
    import synth
    E, H, I, T, K = 6, 256, 128, 3, 2
    host, devt = _experts(6, E, H, I, "blockq", dev)
    x = synth.hidden_states(6, T, H).to(dev)
    ids = torch.tensor([[0, 5], [3, 3], [2, 1]], dtype=torch.int64, device=dev)
    w = torch.tensor([[0.6, 0.4], [0.5, 0.5], [1.0, 0.0]], device=dev)
    got = _run(x, ids, w, devt)
    torch.cuda.synchronize()
    want = omoe.forward_w8a8(_np(x), ids.cpu().numpy(), w.cpu().numpy().astype(np.float64),
                             *(t.numpy() for t in host))
    assert omoe.max_rel_err(_np(got), want) <= TOL


def test_packed_record_views_equal_dense(lib, dev):
    """Expert buffers as strided views into one packed record per expert
    (w13 | w2 | s13 | s2) give bit-identical outputs."""
    import synth
    E, H, I = 10, 2048, 512
    host, devt = _experts(7, E, H, I, "blockq", dev)
    RB = 3_146_496
    rec = torch.zeros((E, RB), dtype=torch.uint8, device=dev)
    o13, o2, os13 = 2 * I * H, 2 * I * H + H * I, 2 * I * H + H * I + 512
    rec[:, :o13] = devt[0].reshape(E, -1)
    rec[:, o13:o2] = devt[2].reshape(E, -1)
    rec[:, o2:os13] = devt[1].reshape(E, -1).view(torch.uint8)
    rec[:, os13:] = devt[3].reshape(E, -1).view(torch.uint8)
    v13 = rec[:, :o13].view(torch.float8_e4m3fn).view(E, 2 * I, H)
    v2 = rec[:, o13:o2].view(torch.float8_e4m3fn).view(E, H, I)
    vs13 = rec[:, o2:os13].view(torch.float32).view(E, 2 * I // 128, H // 128)
    vs2 = rec[:, os13:].view(torch.float32).view(E, H // 128, I // 128)
    x = synth.hidden_states(8, 2).to(dev)
    ids = torch.tensor([[1, 9, 4, 0, 2, 7, 3, 8], [5, 6, 1, 0, 9, 2, 4, 3]], device=dev)
    w = torch.full((2, 8), 0.125, device=dev)
    from fp8_moe import fp8_moe_forward
    a = _run(x, ids, w, devt)
    b = fp8_moe_forward(x, ids, w, v13, vs13, v2, vs2)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_out_of_range_expert_gives_nan_not_a_fault(lib, dev):
    import synth
    E, H, I = 4, 256, 128
    host, devt = _experts(9, E, H, I, "blockq", dev)
    x = synth.hidden_states(9, 2, H).to(dev)
    ids = torch.tensor([[0, 1], [2, 7]], device=dev)
    w = torch.full((2, 2), 0.5, device=dev)
    got = _run(x, ids, w, devt)
    torch.cuda.synchronize()
    assert torch.isfinite(got[0]).all() and torch.isnan(got[1].float()).all()


def test_gemv_id_and_weight_dtypes(lib, dev):
    """The decode kernels read ids (int32/int64) and routing weights
    (float32/bf16) without a branch on the dtype: every combination gives
    the same output as the grouped path; an int64 id whose low word names an
    expert but whose high word is not zero is out of range (NaN row), as
    is -1."""
    import synth
    E, H, I, K = 12, 2048, 512, 8
    host, devt = _experts(17, E, H, I, "blockq", dev)
    for T in (1, 2):
        x = synth.hidden_states(17 + T, T).to(dev)
        rng = np.random.default_rng(T)
        ids = torch.tensor(np.stack([rng.choice(E, K, replace=False) for _ in range(T)]),
                           dtype=torch.int64, device=dev)
        w = torch.rand((T, K), generator=torch.Generator().manual_seed(T)).to(dev)
        w = (w / w.sum(-1, keepdim=True)).to(torch.bfloat16)      # exact in float32 too
        say(f"moe: GEMV dtypes, {T} token(s)")
        outs = [_run(x, i, ww, devt, mode=1) for i in (ids, ids.int()) for ww in (w, w.float())]
        want = _run(x, ids, w.float(), devt, mode=2)
        torch.cuda.synchronize()
        for o in outs:
            assert torch.equal(o, want)
    x = synth.hidden_states(18, 3).to(dev)
    bad = torch.tensor([[0, (1 << 32) + 1], [-1, 3], [4, 5]], dtype=torch.int64, device=dev)
    w = torch.full((3, 2), 0.5, device=dev)
    got = _run(x, bad, w, devt, mode=1)
    good = _run(x[2:], bad[2:], w[2:], devt, mode=1)
    torch.cuda.synchronize()
    assert torch.isnan(got[:2].float()).all()
    assert torch.equal(got[2:], good) and torch.isfinite(good.float()).all()


@pytest.mark.parametrize("K", [1, 3, 7, 15, 16])
def test_gemv_any_top_k_equals_grouped(lib, dev, K):
    """The down kernel pairs experts two to a wave; an odd top_k leaves the
    last wave one expert, and the output still equals the grouped path's
    bit for bit (and the oracle within the bar)."""
    import synth
    E, H, I, T = 20, 2048, 512, 2
    host, devt = _experts(40 + K, E, H, I, "blockq", dev)
    x = synth.hidden_states(40 + K, T).to(dev)
    rng = np.random.default_rng(K)
    ids = torch.tensor(np.stack([rng.choice(E, K, replace=False) for _ in range(T)]), device=dev)
    w = torch.rand((T, K), generator=torch.Generator().manual_seed(K)).to(dev)
    w = w / w.sum(-1, keepdim=True)
    say(f"moe: GEMV top_k {K}")
    a = _run(x, ids, w, devt, mode=1)
    b = _run(x, ids, w, devt, mode=2)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    want = omoe.forward_w8a8(_np(x), ids.cpu().numpy(), w.cpu().numpy().astype(np.float64),
                             *(t.numpy() for t in host))
    assert omoe.max_rel_err(_np(a), want) <= TOL


def test_rejects_cpu_inputs():
    from fp8_moe import fp8_moe_forward
    x = torch.zeros((1, 256), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        fp8_moe_forward(x, torch.zeros((1, 1), dtype=torch.long), torch.ones((1, 1)),
                        torch.zeros((1, 256, 256), dtype=torch.float8_e4m3fn),
                        torch.ones((1, 2, 2)), torch.zeros((1, 256, 128), dtype=torch.float8_e4m3fn),
                        torch.ones((1, 2, 1)))


def test_residual_fusion_equals_bf16_add(lib, dev):
    """out = bf16(residual + bf16(moe)) inside the down kernel equals the MoE
    output followed by a separate bf16 tensor add."""
    import synth
    E, H, I, T, K = 12, 2048, 512, 3, 8
    host, devt = _experts(13, E, H, I, "blockq", dev)
    x = synth.hidden_states(13, T).to(dev)
    res = synth.hidden_states(14, T).to(dev)
    rng = np.random.default_rng(15)
    ids = torch.tensor(np.stack([rng.choice(E, K, replace=False) for _ in range(T)]), device=dev)
    w = torch.full((T, K), 1.0 / K, device=dev)
    plain = _run(x, ids, w, devt)
    fused = torch.empty_like(plain)
    ws = torch.empty(lib.fp8_moe_workspace(T, K, E, H, I), dtype=torch.uint8, device=dev)
    w13, s13, w2, s2 = devt
    lib.fp8_moe_forward(x, ids, w, w13.view(torch.float8_e4m3fn), s13,
                        w2.view(torch.float8_e4m3fn), s2, fused, ws, residual=res)
    fused_x = torch.empty_like(plain)
    lib.fp8_moe_forward(x, ids, w, w13.view(torch.float8_e4m3fn), s13,
                        w2.view(torch.float8_e4m3fn), s2, fused_x, ws, residual=x)
    torch.cuda.synchronize()
    assert torch.equal(fused, res + plain)
    assert torch.equal(fused_x, x + plain)
