"""The routed-expert module and router the offload hooks attach to.

Upstream fish-speech's `MoEExperts` (moe.py:87-135 as described in
notes/01-static-findings.md:84-138) is not part of the reference tree; the
hooks in bin/offload.py and bin/devcache.py only rely on this surface:

  * attributes num_experts, w13_weight [E, 2I, H] and w2_weight [E, H, I]
    (float8_e4m3fn), w13_scale_inv [E, 2I/128, H/128] and w2_scale_inv
    [E, H/128, I/128] (float32), registered as BUFFERS, not Parameters, so a
    module whose experts live in host memory still counts as single-device
    for graph capture (notes/01-static-findings.md:166-185);
  * forward(x, topk_ids, topk_weights) -> [T, H], replaced at class level by
    install_offload / install_dev_cache (bin/offload.py:702-704,
    bin/devcache.py:300);
  * select_fp8(w, index): index float8 storage through a uint8 view
    (notes/13-non-ada-gpus.md:31-35).

`SparseMoE` is the block that owns the router gate (nn.Linear(H, E), bf16)
and calls the experts, and `route` is the router itself (HIP kernel).
"""
from __future__ import annotations

import torch
from torch import nn

import hipfetch
from fp8_moe import fp8_moe_forward

F8 = torch.float8_e4m3fn


def select_fp8(w: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """w[index] for float8 storage (advanced indexing has no float8 kernel)."""
    return w.view(torch.uint8)[index].view(w.dtype)


class MoEExperts(nn.Module):
    """E routed experts of one layer, FP8 weights with 128x128 block scales."""

    def __init__(self, num_experts: int, hidden: int, intermediate: int, fp8: bool = True,
                 device=None):
        super().__init__()
        if not fp8:
            raise ValueError("only FP8 expert storage is supported")
        self.num_experts = num_experts
        self.hidden = hidden
        self.intermediate = intermediate
        self.fp8 = True
        dev = torch.device(device) if device is not None else torch.device("cpu")
        self.register_buffer("w13_weight",
                             torch.zeros((num_experts, 2 * intermediate, hidden), dtype=F8, device=dev))
        self.register_buffer("w2_weight",
                             torch.zeros((num_experts, hidden, intermediate), dtype=F8, device=dev))
        self.register_buffer("w13_scale_inv",
                             torch.ones((num_experts, 2 * intermediate // 128, hidden // 128),
                                        dtype=torch.float32, device=dev))
        self.register_buffer("w2_scale_inv",
                             torch.ones((num_experts, hidden // 128, intermediate // 128),
                                        dtype=torch.float32, device=dev))

    def forward(self, x: torch.Tensor, topk_ids: torch.Tensor,
                topk_weights: torch.Tensor) -> torch.Tensor:
        """All experts resident on the GPU: run the HIP kernels directly."""
        if self.w13_weight.device.type != "cuda":
            raise RuntimeError("expert weights are in host memory; install the offload hooks "
                               "(offload.install_offload / devcache.install_dev_cache)")
        return fp8_moe_forward(x, topk_ids, topk_weights, self.w13_weight, self.w13_scale_inv,
                               self.w2_weight, self.w2_scale_inv)

    # the class-level hooks keep a handle on the resident-weight forward
    _stock_forward = forward


def route(x: torch.Tensor, gate_weight: torch.Tensor, top_k: int = 8,
          bias: torch.Tensor | None = None, ids_dtype=torch.int64,
          weights_dtype=torch.float32, out=None, logit_dtype: str = "bf16"):
    """Router on the GPU: logits = x . W^T (+bias), top-k, renormalised softmax.

    x [T, H] bf16, gate_weight [E, H] bf16.  The logits are rounded to bf16
    as the output of the model's bf16 nn.Linear gate is (logit_dtype "f32"
    keeps float32 logits).  Returns (topk_ids [T, k], topk_weights [T, k],
    logits [T, E] float32).  `out` may be a preallocated (ids, weights,
    logits) triple (graph capture)."""
    lib = hipfetch.require()
    T = x.shape[0]
    E = gate_weight.shape[0]
    if out is None:
        ids = torch.empty((T, top_k), dtype=ids_dtype, device=x.device)
        wts = torch.empty((T, top_k), dtype=weights_dtype, device=x.device)
        logits = torch.empty((T, E), dtype=torch.float32, device=x.device)
    else:
        ids, wts, logits = out
    lib.router_topk(x.contiguous(), gate_weight.contiguous(), bias, top_k, logits, ids, wts,
                    logit_dtype=logit_dtype)
    return ids, wts, logits


class SparseMoE(nn.Module):
    """Router gate + routed experts (the upstream MoE block's routed half)."""

    def __init__(self, num_experts: int, hidden: int, intermediate: int, top_k: int = 8,
                 device=None, expert_device=None):
        super().__init__()
        self.top_k = top_k
        self.gate = nn.Linear(hidden, num_experts, bias=False, device=device,
                              dtype=torch.bfloat16)
        self.experts = MoEExperts(num_experts, hidden, intermediate,
                                  device=expert_device if expert_device is not None else device)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        ids, wts, _ = route(x, self.gate.weight, self.top_k)
        return self.experts(x, ids, wts)
