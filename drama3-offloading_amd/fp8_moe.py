"""fp8_moe_forward: the W8A8 block-FP8 routed-expert FFN on gfx950.

Same call shape as upstream's Triton `fp8_moe_forward(x, topk_ids,
topk_weights, w13, s13, w2, s2)` as the reference calls it
(bin/devcache.py:275-277, bin/offload.py:177,239,340,388,449): the expert
count is read from w13.shape[0], so a renumbered subset or the whole device
cache with slot ids is legal (bin/offload.py:9-11).

Everything runs in libmoeoffload's HIP kernels; there is no CPU or Triton
path, and a missing library raises.
"""
from __future__ import annotations

import torch

import hipfetch

# kernel choice: automatic (per-pair GEMV up to 16 tokens, grouped beyond),
# per-pair GEMV, grouped -- all W8A8 (activations quantised to e4m3 per 128
# columns) -- and the per-pair GEMV with bf16 activations (W8A16: the
# numerics of the dequantise-then-matmul path, bin/offload.py's CPU experts)
MODE_AUTO, MODE_GEMV, MODE_GROUPED, MODE_GEMV_A16 = 0, 1, 2, 3


def workspace_bytes(tokens: int, top_k: int, n_experts: int, hidden: int, inter: int) -> int:
    return hipfetch.require().fp8_moe_workspace(tokens, top_k, n_experts, hidden, inter)


def fp8_moe_forward(x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                    w13: torch.Tensor, s13: torch.Tensor, w2: torch.Tensor, s2: torch.Tensor,
                    *, out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                    mode: int = MODE_AUTO, layout: int = hipfetch.LAYOUT_ROWS) -> torch.Tensor:
    """x [T, H] bf16; topk_ids [T, K] int32/int64; topk_weights [T, K] f32/bf16;
    w13 [n, 2I, H] and w2 [n, H, I] float8_e4m3fn (or uint8 views of them);
    s13 [n, 2I/128, H/128], s2 [n, H/128, I/128] float32.  Returns [T, H] bf16.

    `out` and `workspace` may be passed in (preallocated, e.g. for graph
    capture); otherwise they are allocated from torch's caching allocator.
    `layout`: byte order of w13/w2 -- row-major as in the checkpoint
    (default), or hipfetch.LAYOUT_TILES for views of packed records.
    `mode` MODE_GEMV_A16 keeps the activations in bf16 (x as given,
    SiLU(gate) * up rounded to bf16) instead of quantising them to e4m3."""
    lib = hipfetch.require()
    if not x.is_cuda:
        raise RuntimeError("fp8_moe_forward runs on the GPU only; x is on "
                           f"{x.device} (there is no CPU path)")
    if x.dtype != torch.bfloat16 or x.dim() != 2 or not x.is_contiguous():
        raise ValueError("x must be a contiguous [T, H] bfloat16 tensor")
    if topk_ids.dim() != 2 or topk_ids.shape[0] != x.shape[0]:
        raise ValueError(f"topk_ids must be [T, K] with T = {x.shape[0]}")
    if topk_weights.shape != topk_ids.shape:
        raise ValueError("topk_weights must have the shape of topk_ids")
    ids = topk_ids if topk_ids.is_contiguous() else topk_ids.contiguous()
    if ids.dtype not in (torch.int32, torch.int64):
        ids = ids.to(torch.int64)
    wts = topk_weights if topk_weights.is_contiguous() else topk_weights.contiguous()
    if wts.dtype not in (torch.float32, torch.bfloat16):
        wts = wts.to(torch.float32)
    T, H = x.shape
    K = ids.shape[1]
    n, I2, H2 = w13.shape
    if H2 != H or w2.shape[0] != n or w2.shape[1] != H or w2.shape[2] * 2 != I2:
        raise ValueError(f"w13 {tuple(w13.shape)} / w2 {tuple(w2.shape)} do not match x [T, {H}]")
    inter = w2.shape[2]
    if s13.dtype != torch.float32 or s2.dtype != torch.float32:
        raise ValueError("s13/s2 must be float32 scale_inv blocks")
    if tuple(s13.shape[1:]) != (I2 // 128, H // 128) or tuple(s2.shape[1:]) != (H // 128, inter // 128):
        raise ValueError(f"scale shapes {tuple(s13.shape)} / {tuple(s2.shape)} do not match "
                         "128x128 blocks")
    # a host address handed to a kernel would fault the device
    for t in (topk_ids, topk_weights, w13, s13, w2, s2):
        if t.device != x.device:
            raise ValueError(f"ids, weights and expert buffers must be on {x.device}, "
                             f"got one on {t.device}")
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=x.device)
    need = lib.fp8_moe_workspace(T, K, n, H, inter)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    lib.fp8_moe_forward(x, ids, wts, w13, s13, w2, s2, out, workspace, mode, layout=layout)
    return out
