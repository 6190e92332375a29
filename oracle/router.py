"""Top-k-of-E router: linear -> softmax -> top-k -> renormalise.

Oracle (test infrastructure).  Upstream's router is an nn.Linear(2048, 256)
gate, softmax, top-8 and renormalisation (`norm_topk_prob`), with no noise
and no auxiliary loss at inference (moe.py:217-220 as described in
notes/01-static-findings.md:133-138; config notes/drama3-config.json
text_config num_experts 256, num_experts_per_tok 8, norm_topk_prob true).

The reference tree fixes neither the logit precision nor the tie-break.
This build's contract, which the HIP kernel follows exactly:
  * logit[t, e] = float32( sum_k x[t,k] * W[e,k] ), every bf16 x bf16
    product exact and the sum accumulated in float64 before one rounding to
    float32; an optional float32 bias is then added in float32;
  * selection by descending logit, ties to the LOWER expert index;
  * weights = softmax over the selected logits (identical to softmax over
    all E followed by renormalisation over the selected k).
Agreement with upstream's own rounding is "parity unpinned".
"""
from __future__ import annotations

import numpy as np

_F32 = np.float32


def logits(x, w, bias=None) -> np.ndarray:
    """x [T, H] float32 (bf16 values), w [E, H] float32 (bf16 values)."""
    lg = (np.asarray(x, np.float64) @ np.asarray(w, np.float64).T).astype(_F32)
    if bias is not None:
        lg = (lg + np.asarray(bias, _F32)[None, :]).astype(_F32)
    return lg


def topk(lg: np.ndarray, k: int):
    """Descending logit, ties to the lower index.  Returns (ids int32 [T,k],
    weights float64 [T,k])."""
    lg = np.asarray(lg, _F32)
    T, E = lg.shape
    ids = np.empty((T, k), np.int32)
    wts = np.empty((T, k), np.float64)
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-float(lg[t, e]), e))[:k]
        ids[t] = order
        sel = lg[t, order].astype(np.float64)
        ex = np.exp(sel - sel.max())
        wts[t] = ex / ex.sum()
    return ids, wts


def route(x, w, k: int = 8, bias=None):
    lg = logits(x, w, bias)
    ids, wts = topk(lg, k)
    return ids, wts, lg
