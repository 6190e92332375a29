"""Top-k-of-E router: linear -> softmax -> top-k -> renormalise.

Oracle (test infrastructure).  Upstream's router is an nn.Linear(2048, 256)
gate in bf16, a plain softmax, top-8 and renormalisation (`norm_topk_prob`),
with no noise and no auxiliary loss at inference (moe.py:217-220 as
described in notes/01-static-findings.md:133-138; config
notes/drama3-config.json text_config num_experts 256, num_experts_per_tok 8,
norm_topk_prob true).

The reference tree fixes neither the logit precision nor the tie-break.
This build's contract, which the HIP kernel follows exactly:
  * s[t, e] = sum_k x[t,k] * W[e,k], every bf16 x bf16 product exact and the
    sum accumulated in float64;
  * logit = s rounded once, either to bf16 (logit_dtype "bf16", the default:
    the output of a bf16 nn.Linear is a bf16 tensor, rounded to nearest even)
    or to float32 ("f32"); an optional float32 bias is then added in float32;
  * selection by descending logit, ties to the LOWER expert index (bf16
    logits tie far more often than float32 ones);
  * weights = softmax over the selected logits (identical to softmax over
    all E followed by renormalisation over the selected k).
The bf16 logits are pinned against torch's own bf16 F.linear on the CPU
(equal but for rare one-ulp differences from torch's float32 accumulation);
agreement with upstream's GPU gate is "parity unpinned".
"""
from __future__ import annotations

import numpy as np

_F32 = np.float32


def bf16_round(d) -> np.ndarray:
    """Nearest bf16 (ties to even) of float64 values, returned as float32.

    Works on the float64 bit pattern: bf16 keeps 7 of float64's 52 fraction
    bits, so the low 45 bits are rounded away, half to even, by integer
    addition (a carry into the exponent is the correct round-up).  Values
    below 2^-126 (bf16's subnormal range) are rounded on its 2^-133 grid
    instead.  Finite inputs only."""
    d = np.asarray(d, np.float64)
    bits = d.view(np.uint64)
    low = np.uint64((1 << 45) - 1)
    odd = (bits >> np.uint64(45)) & np.uint64(1)
    r = ((bits + np.uint64((1 << 44) - 1) + odd) & ~low).view(np.float64)
    tiny = np.abs(d) < 2.0 ** -126
    if np.any(tiny):
        r = np.where(tiny, np.round(d * 2.0 ** 133) * 2.0 ** -133, r)
    return r.astype(_F32)


def logits(x, w, bias=None, logit_dtype: str = "bf16") -> np.ndarray:
    """x [T, H] float32 (bf16 values), w [E, H] float32 (bf16 values)."""
    s = np.asarray(x, np.float64) @ np.asarray(w, np.float64).T
    if logit_dtype == "bf16":
        lg = bf16_round(s)
    elif logit_dtype == "f32":
        lg = s.astype(_F32)
    else:
        raise ValueError(f"logit_dtype must be 'bf16' or 'f32', got {logit_dtype!r}")
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


def route(x, w, k: int = 8, bias=None, logit_dtype: str = "bf16"):
    lg = logits(x, w, bias, logit_dtype)
    ids, wts = topk(lg, k)
    return ids, wts, lg
