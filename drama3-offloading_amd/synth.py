"""Seeded synthetic Drama-3-shaped inputs (there is no checkpoint here).

Shapes: hidden 2048, expert intermediate 512, 256 experts, top-8, 40 layers
(notes/drama3-config.json text_config).  Recipes:

  "blockq"  weights ~ N(0, 0.02); per 128x128 block scale_inv = amax/448 and
            q = e4m3fn(w / scale_inv), round-to-nearest-even (the seeded
            single-layer workload's recipe)
  "devtest" the reference's device-cache test recipe: q = e4m3fn(randn*0.2)
            directly, scales U(0.05, 0.15) (bin/test_devcache.py:33-37)

Every expert has its own generator seeded from (seed, layer, expert), so any
expert can be regenerated alone and the CPU and GPU tests agree on bytes.
"""
from __future__ import annotations

import numpy as np
import torch

F8 = torch.float8_e4m3fn
HIDDEN, INTER, N_EXPERTS, TOP_K, LAYERS = 2048, 512, 256, 8, 40


def _seed(seed: int, layer: int, expert: int) -> int:
    return (seed * 1_000_003 + layer * 10_007 + expert * 101 + 17) % (2**63 - 1)


def quantize_blocks(w: torch.Tensor, block: int = 128):
    """[..., R, C] float32 -> (uint8 e4m3 codes, float32 scale_inv [..., R/128, C/128])."""
    *lead, R, C = w.shape
    b = w.reshape(*lead, R // block, block, C // block, block)
    amax = b.abs().amax(dim=(-3, -1))
    scale = amax / 448.0
    scale = torch.where(amax == 0, torch.ones_like(scale), scale)
    q = (b / scale.unsqueeze(-1).unsqueeze(-3)).to(F8)
    return q.view(torch.uint8).reshape(*lead, R, C), scale.to(torch.float32)


def expert_tensors(seed: int, layer: int, expert: int, hidden: int = HIDDEN, inter: int = INTER,
                   recipe: str = "blockq", std: float = 0.02, device="cpu"):
    """One expert: (w13 uint8 [2I, H], s13 f32 [2I/128, H/128], w2 uint8 [H, I],
    s2 f32 [H/128, I/128]); rows 0..I-1 of w13 are gate, I..2I-1 up."""
    g = torch.Generator(device=device).manual_seed(_seed(seed, layer, expert))
    if recipe == "blockq":
        w13 = torch.randn((2 * inter, hidden), generator=g, device=device) * std
        w2 = torch.randn((hidden, inter), generator=g, device=device) * std
        q13, s13 = quantize_blocks(w13)
        q2, s2 = quantize_blocks(w2)
        return q13, s13, q2, s2
    if recipe == "devtest":
        q13 = (torch.randn((2 * inter, hidden), generator=g, device=device) * 0.2).to(F8)
        q2 = (torch.randn((hidden, inter), generator=g, device=device) * 0.2).to(F8)
        s13 = torch.rand((2 * inter // 128, hidden // 128), generator=g, device=device) * 0.1 + 0.05
        s2 = torch.rand((hidden // 128, inter // 128), generator=g, device=device) * 0.1 + 0.05
        return q13.view(torch.uint8), s13, q2.view(torch.uint8), s2
    raise ValueError(f"unknown recipe {recipe!r}")


def fill_experts(experts, seed: int, layer: int = 0, recipe: str = "blockq",
                 gen_device="cpu") -> None:
    """Fill an MoEExperts module's four buffers in place."""
    E = experts.num_experts
    H = experts.w13_weight.shape[2]
    I = experts.w2_weight.shape[2]
    with torch.no_grad():
        for e in range(E):
            q13, s13, q2, s2 = expert_tensors(seed, layer, e, H, I, recipe, device=gen_device)
            experts.w13_weight.view(torch.uint8)[e].copy_(q13)
            experts.w13_scale_inv[e].copy_(s13)
            experts.w2_weight.view(torch.uint8)[e].copy_(q2)
            experts.w2_scale_inv[e].copy_(s2)


def hidden_states(seed: int, tokens: int, hidden: int = HIDDEN, device="cpu") -> torch.Tensor:
    g = torch.Generator(device=device).manual_seed(_seed(seed, 999_983, 1))
    return torch.randn((tokens, hidden), generator=g, device=device).to(torch.bfloat16)


def router_weight(seed: int, layer: int = 0, n_experts: int = N_EXPERTS, hidden: int = HIDDEN,
                  device="cpu") -> torch.Tensor:
    g = torch.Generator(device=device).manual_seed(_seed(seed, layer, 999_979))
    return (torch.randn((n_experts, hidden), generator=g, device=device) * 0.02).to(torch.bfloat16)


def zipf_probs(n: int = N_EXPERTS, s: float = 1.1) -> np.ndarray:
    p = np.arange(1, n + 1, dtype=np.float64) ** -s
    return p / p.sum()


def zipf_miss_list(rng: np.random.Generator, length: int, n: int = N_EXPERTS,
                   s: float = 1.1) -> np.ndarray:
    """`length` distinct expert ids, drawn without replacement with
    p(rank r) ~ r^-s over a fresh random permutation of the experts."""
    perm = rng.permutation(n)
    picks = rng.choice(n, size=length, replace=False, p=zipf_probs(n, s))
    return perm[picks].astype(np.int32)


def decode_route_bias(rng: np.random.Generator, steps: int, layers: int = LAYERS,
                      n: int = N_EXPERTS, s: float = 1.1, drift_every: int = 50) -> np.ndarray:
    """Per-step, per-layer router bias [steps, layers, n] float32 making top-8
    routing follow a per-layer Zipf(s) popularity over a permutation that is
    redrawn every `drift_every` steps: log-popularity plus Gumbel noise, so
    the top-8 of (bias + small logits) is a draw without replacement from
    the Zipf law."""
    logp = np.log(zipf_probs(n, s))
    out = np.empty((steps, layers, n), dtype=np.float32)
    perms = None
    for t in range(steps):
        if t % drift_every == 0:
            perms = [rng.permutation(n) for _ in range(layers)]
        for l in range(layers):
            lp = np.empty(n)
            lp[perms[l]] = logp
            out[t, l] = lp + rng.gumbel(size=n)
    return out
