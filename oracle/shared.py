"""The MoE block's gated shared expert and the decode finiteness guard.

Oracle (test infrastructure).

Drama-3's MoE block passes every token through a dense bf16 shared expert
besides the 8 routed ones, scales it by a sigmoid gate and adds it to the
routed output (notes/drama3-config.json:215-216: shared_expert_gate true,
shared_expert_intermediate_size 512; notes/01-static-findings.md:80-82;
checkpoint tensors layers.N.mlp.shared_expert.{gate,up,down}_proj.weight
[512,2048]/[512,2048]/[2048,512] and layers.N.mlp.shared_expert_gate.weight
[1,2048], all BF16, tests/golden/drama3_mlp_headers.json.gz).  The module is
upstream's and is not in the reference, so its exact form is the
conventional one for a gated shared expert, in the op order of bf16 torch
modules: every Linear accumulates in float32 and rounds its output to bf16,
every elementwise op rounds its float32 result to bf16.

    g = bf16(x Wg^T)  u = bf16(x Wu^T)  a = bf16(bf16(silu(g)) * u)
    d = bf16(a Wd^T)  s = bf16(sigmoid(bf16(x wsg^T)))  sh = bf16(s * d)
    block = bf16(routed + sh)          out = bf16(residual + block)

Sums here run in float64 and are rounded to float32 first, then to bf16 (a
float32 accumulator's result is within float32 rounding of the float64 sum).
"""
from __future__ import annotations

import numpy as np

from .fp8 import bf16_round

_F32 = np.float32


def _linear(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """bf16(x @ w^T), x [T, K], w [N, K] (bf16 values as float32)."""
    return bf16_round((x.astype(np.float64) @ w.astype(np.float64).T).astype(_F32))


def _silu(v: np.ndarray) -> np.ndarray:
    v = v.astype(_F32)
    return (v / (_F32(1.0) + np.exp(-v))).astype(_F32)


def _sigmoid(v: np.ndarray) -> np.ndarray:
    v = v.astype(_F32)
    return (_F32(1.0) / (_F32(1.0) + np.exp(-v))).astype(_F32)


def gate_up(x, w_gate, w_up, w_sgate):
    """(act [T, Is], sig [T]) of the shared expert's first half."""
    x = np.asarray(x, _F32)
    g = _linear(x, np.asarray(w_gate, _F32))
    u = _linear(x, np.asarray(w_up, _F32))
    a = bf16_round((bf16_round(_silu(g)) * u).astype(_F32))
    z = _linear(x, np.asarray(w_sgate, _F32).reshape(1, -1))[:, 0]
    return a, bf16_round(_sigmoid(z))


def down(act, sig, w_down, routed=None, residual=None):
    """bf16(residual + bf16(routed + bf16(sig * bf16(act Wd^T))))."""
    d = _linear(np.asarray(act, _F32), np.asarray(w_down, _F32))
    v = bf16_round((np.asarray(sig, _F32)[:, None] * d).astype(_F32))
    if routed is not None:
        v = bf16_round((np.asarray(routed, _F32) + v).astype(_F32))
    if residual is not None:
        v = bf16_round((np.asarray(residual, _F32) + v).astype(_F32))
    return v


def shared_expert(x, w_gate, w_up, w_down, w_sgate, routed=None, residual=None):
    a, s = gate_up(x, w_gate, w_up, w_sgate)
    return down(a, s, w_down, routed, residual)


def all_finite(x) -> bool:
    """torch.isfinite(x).all() of the decode graph's guard
    (generate.py:376-377, quoted in notes/botnotes/lm-head-inf-sentinel.md:18-28)."""
    return bool(np.isfinite(np.asarray(x, np.float64)).all())
