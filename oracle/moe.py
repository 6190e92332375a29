"""The routed-expert FFN in the two numerics this path is checked against.

Oracle (test infrastructure).

Shapes follow upstream `fp8_moe_forward(x, topk_ids, topk_weights, w13, s13,
w2, s2)` as called at bin/devcache.py:275-277 and bin/offload.py:239:
  x        [T, H]        bf16 (passed here as float32 values)
  topk_ids [T, K]        expert index into the first axis of w13/w2
  topk_w   [T, K]        routing weights
  w13      [n, 2I, H]    e4m3 codes; rows 0..I-1 gate, I..2I-1 up
  s13      [n, 2I/128, H/128] float32 scale_inv
  w2       [n, H, I]     e4m3 codes
  s2       [n, H/128, I/128]  float32 scale_inv
  -> out   [T, H]        bf16

Per (t, k) pair with e = topk_ids[t, k]:
  g, u = (W13[e] @ x_t) split in halves;  a = SiLU(g) * u
  y = W2[e] @ a;  out_t = sum_k topk_w[t, k] * y   (notes/13-non-ada-gpus.md:31-53
  for the dequantise path; the gate/up row order is the conventional one and
  is not confirmed inside the reference, bin/offload.py:9-11 only fixes that
  the expert axis is w13.shape[0]).

`forward_w8a8` is the contract of this build's HIP kernels: activations are
quantised per token per 128 columns (oracle.fp8.quantize_activation) before
each of the two products, each 128-wide block product is exact, block results
are scaled by weight_scale_inv * activation_scale and summed.  The reference's
GPU kernel is upstream Triton W8A8 with dynamic activation quant, which is not
in the reference tree, so agreement with IT is "parity unpinned"; agreement
with this restatement is what the GPU tests enforce.

`forward_w8a16` is the reference's CPU path: dequantise the selected experts
with their block scales, then ordinary matmuls (notes/13-non-ada-gpus.md:37-53,
bin/bench_copy.py:16,40).  It differs from W8A8 by the activation
quantisation error (a few percent of an output's magnitude), which the tests
measure and report.
"""
from __future__ import annotations

import numpy as np

from . import fp8

_F32 = np.float32


def silu(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, dtype=np.float64)
    return v / (1.0 + np.exp(-v))


def _block_gemv_w8a8(wq: np.ndarray, ws: np.ndarray, aq: np.ndarray, as_: np.ndarray,
                     block: int = 128) -> np.ndarray:
    """Exact per-block products, float64 scaling and accumulation.

    wq [R, D] codes, ws [R/128, D/128] scale_inv, aq [D] codes, as_ [D/128].
    Returns float64 [R] = sum_g ws[r//128, g] * as_[g] * sum_{k in g} w[r,k] a[k].
    A product of two e4m3 values has an 8-bit significand and spans at most
    2^-18..2^18, so float64 sums of 128 of them are exact.
    """
    R, D = wq.shape
    G = D // block
    wv = fp8.decode(wq).reshape(R, G, block)
    av = fp8.decode(aq).reshape(G, block)
    blk = np.einsum("rgk,gk->rg", wv, av)               # exact in float64
    scale = np.repeat(np.asarray(ws, np.float64), block, axis=0)[:R] * \
        np.asarray(as_, np.float64)[None, :]
    return (blk * scale).sum(axis=1)


def expert_w8a8(x_row: np.ndarray, w13q, s13, w2q, s2) -> np.ndarray:
    """One expert on one token, W8A8.  Returns float64 y [H]."""
    H = x_row.shape[0]
    I2 = w13q.shape[0]
    I = I2 // 2
    xq, xs = fp8.quantize_activation(np.asarray(x_row, _F32)[None, :])
    h = _block_gemv_w8a8(w13q, s13, xq[0], xs[0])
    # the kernels keep the gate/up results and SiLU*mul in float32
    h32 = h.astype(_F32)
    a = (silu(h32[:I]) * h32[I:].astype(np.float64)).astype(_F32)
    aq, as_ = fp8.quantize_activation(a[None, :])
    y = _block_gemv_w8a8(w2q, s2, aq[0], as_[0])
    assert y.shape[0] == H
    return y


def forward_w8a8(x, topk_ids, topk_w, w13q, s13, w2q, s2) -> np.ndarray:
    """Full W8A8 MoE forward.  Returns float32 values rounded to bf16."""
    x = np.asarray(x, _F32)
    ids = np.asarray(topk_ids, np.int64)
    tw = np.asarray(topk_w, np.float64)
    T, K = ids.shape
    out = np.zeros((T, x.shape[1]), np.float64)
    for t in range(T):
        for k in range(K):
            e = ids[t, k]
            y = expert_w8a8(x[t], w13q[e], s13[e], w2q[e], s2[e]).astype(_F32)
            out[t] += tw[t, k] * y.astype(np.float64)
    return fp8.bf16_round(out.astype(_F32))


def forward_w8a8_unrounded(x, topk_ids, topk_w, w13q, s13, w2q, s2) -> np.ndarray:
    """Same as forward_w8a8 but returns the float64 sum before bf16 rounding."""
    x = np.asarray(x, _F32)
    ids = np.asarray(topk_ids, np.int64)
    tw = np.asarray(topk_w, np.float64)
    T, K = ids.shape
    out = np.zeros((T, x.shape[1]), np.float64)
    for t in range(T):
        for k in range(K):
            e = ids[t, k]
            y = expert_w8a8(x[t], w13q[e], s13[e], w2q[e], s2[e]).astype(_F32)
            out[t] += tw[t, k] * y.astype(np.float64)
    return out


def forward_w8a16(x, topk_ids, topk_w, w13q, s13, w2q, s2) -> np.ndarray:
    """Dequantise-then-matmul MoE forward (the reference's CPU path), float64.

    Returns float32 values rounded to bf16.
    """
    x = np.asarray(x, np.float64)
    ids = np.asarray(topk_ids, np.int64)
    tw = np.asarray(topk_w, np.float64)
    T, K = ids.shape
    I = w13q.shape[1] // 2
    out = np.zeros((T, x.shape[1]), np.float64)
    cache = {}
    for t in range(T):
        for k in range(K):
            e = int(ids[t, k])
            if e not in cache:
                cache[e] = (fp8.dequantize_blocks(w13q[e], s13[e]),
                            fp8.dequantize_blocks(w2q[e], s2[e]))
            w13, w2 = cache[e]
            h = w13 @ x[t]
            a = silu(h[:I]) * h[I:]
            out[t] += tw[t, k] * (w2 @ a)
    return fp8.bf16_round(out.astype(_F32))


def max_rel_err(got, want) -> float:
    """max |got - want| / max |want| (normwise), the tolerance metric used by
    every MoE-output check in this build."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.abs(want).max()
    return float(np.abs(got - want).max() / den) if den > 0 else float(np.abs(got).max())
