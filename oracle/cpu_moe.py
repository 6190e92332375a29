"""The reference's CPU MoE path, timed as the bench's CPU baseline.

Oracle (test infrastructure; only bench.py's cpu_baseline leg runs it).

Upstream's non-FP8-compute path gathers the routed experts, dequantises them
per 128x128 block and multiplies with ordinary matmuls (`expert_weights` ->
`dequantize_fp8_blocks(select_fp8(w, index), scale_inv[index], dtype)`, then
`forward_gathered` bmm; notes/13-non-ada-gpus.md:37-53).  Restated here with
torch on the host cores in float32, reading the packed records straight out
of the page-locked pool the GPU fetches from.  One decode step mirrors the
GPU harness: per layer a [2048, 2048] stub matmul, the router, then the
8 routed experts.

The pool stores w13/w2 in the GPU kernels' MFMA tile order; the reference's
host tensors are row-major.  The selected records are put back in row order
before dequantisation and that permutation is timed apart (UNTILE_SECONDS)
and left out of the reported times: it is a cost of this storage format,
not of the reference's CPU path.
"""
from __future__ import annotations

import time

import torch


def dequantize_fp8_blocks(q_u8: torch.Tensor, scale_inv: torch.Tensor,
                          dtype=torch.float32) -> torch.Tensor:
    """q [n, R, C] uint8 e4m3 codes, scale_inv [n, R/128, C/128] -> [n, R, C]."""
    w = q_u8.view(torch.float8_e4m3fn).to(dtype)
    s = scale_inv.to(dtype).repeat_interleave(128, dim=-2).repeat_interleave(128, dim=-1)
    return w * s


# Seconds spent putting tile-ordered records back in row order (excluded
# from the timings below); reset by each timing function.
UNTILE_SECONDS = 0.0


def _row_order(b: torch.Tensor) -> torch.Tensor:
    """[n, R, K] uint8 in MFMA tile order (row group, K-block, 1 KiB half,
    16-byte unit 16q + r, byte; hostpool.to_tiles) -> row-major."""
    n, R, K = b.shape
    return (b.reshape(n, R // 16, K // 128, 2, 4, 16, 16)
            .permute(0, 1, 5, 2, 4, 3, 6).reshape(n, R, K))


def moe_forward_cpu(x: torch.Tensor, ids: torch.Tensor, wts: torch.Tensor,
                    records: torch.Tensor, layout) -> torch.Tensor:
    """x [T, H] float32, ids/wts [T, K], records uint8 [E, record_bytes]."""
    global UNTILE_SECONDS
    T, K = ids.shape
    H, I = layout.hidden, layout.inter
    uniq, inv = torch.unique(ids, return_inverse=True)
    rec = records[uniq]                                          # CPU gather (select_fp8)
    n = rec.shape[0]
    q13 = rec[:, :layout.off_w2].view(n, 2 * I, H)
    q2 = rec[:, layout.off_w2:layout.off_s13].view(n, H, I)
    if getattr(layout, "tiled", False):
        t0 = time.perf_counter()
        q13, q2 = _row_order(q13), _row_order(q2)
        UNTILE_SECONDS += time.perf_counter() - t0
    w13 = dequantize_fp8_blocks(q13, rec[:, layout.off_s13:layout.off_s2].contiguous()
                                .view(torch.float32).view(n, 2 * I // 128, H // 128))
    w2 = dequantize_fp8_blocks(q2, rec[:, layout.off_s2:layout.payload_bytes].contiguous()
                               .view(torch.float32).view(n, H // 128, I // 128))
    flat = inv.reshape(-1)
    xs = x.repeat_interleave(K, dim=0).unsqueeze(-1)             # [T*K, H, 1]
    h = torch.bmm(w13[flat], xs).squeeze(-1)                     # [T*K, 2I]
    a = torch.nn.functional.silu(h[:, :I]) * h[:, I:]
    y = torch.bmm(w2[flat], a.unsqueeze(-1)).squeeze(-1)         # [T*K, H]
    return (y.view(T, K, H) * wts.unsqueeze(-1)).sum(1)


def decode_step_cpu(x, w_stub, gate, bias, records, layout, top_k=8, layers=None):
    """One batch-1 decode step over `layers` layers (all by default);
    w_stub [L, out, in] as the GPU harness holds it: h = x w_stub[l]^T."""
    L = w_stub.shape[0] if layers is None else layers
    for l in range(L):
        h = x @ w_stub[l].T
        logits = h @ gate[l].T + bias[l]
        val, ids = torch.topk(logits, top_k, dim=-1)
        wts = torch.softmax(val, dim=-1)
        x = h + moe_forward_cpu(h, ids, wts, records[l], layout)
    return x


def time_decode(w_stub, gate, bias, records, layout, x0, budget_s: float = 25.0,
                top_k: int = 8, max_tokens: int = 20):
    """Run whole layers, token after token, until ~budget_s of CPU work or
    max_tokens tokens; bias [L, E], or [S, L, E] for token t to take the
    routing bias of schedule step t % S.  Returns (seconds per token,
    layers run, threads)."""
    global UNTILE_SECONDS
    L = w_stub.shape[0]
    per_step = bias.dim() == 3
    step_bias = (lambda t: bias[t % bias.shape[0]]) if per_step else (lambda t: bias)
    x = x0
    # warm-up one layer
    decode_step_cpu(x, w_stub[:1], gate[:1], step_bias(0)[:1], records[:1], layout, top_k)
    UNTILE_SECONDS = 0.0
    t0 = time.perf_counter()
    done = 0
    while True:
        l = done % L
        if l == 0:
            x = x0                      # every token starts from the same input state
        b = step_bias(done // L)
        x = decode_step_cpu(x, w_stub[l:l + 1], gate[l:l + 1], b[l:l + 1],
                            records[l:l + 1], layout, top_k)
        done += 1
        el = time.perf_counter() - t0 - UNTILE_SECONDS
        if (el >= budget_s and done >= 4) or done >= max_tokens * L:
            break
    per_layer = el / done
    return per_layer * L, done, torch.get_num_threads()


def median_seconds(fn, iters: int = 20, warmup: int = 3) -> float:
    """Median wall time of fn() over `iters` runs after `warmup` runs, less
    the record untiling each run did."""
    global UNTILE_SECONDS
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(iters):
        UNTILE_SECONDS = 0.0
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0 - UNTILE_SECONDS)
    ts.sort()
    return ts[len(ts) // 2]


def time_single_layer(x, w_stub, gate, bias, records, layout, top_k: int = 8,
                      iters: int = 20, threads: int | None = None) -> float:
    """Median seconds of one decode layer (stub, router, 8-expert
    dequantise-then-matmul MoE) on `threads` host threads."""
    old = torch.get_num_threads()
    if threads:
        torch.set_num_threads(threads)
    try:
        return median_seconds(lambda: decode_step_cpu(x, w_stub[:1], gate[:1], bias[:1],
                                                      records[:1], layout, top_k), iters)
    finally:
        torch.set_num_threads(old)


def time_gather(records, ids, iters: int = 20) -> float:
    """Median seconds of gathering the routed records on the host (the CPU
    side of the reference's "gather" copy mode, bin/offload.py:181-185)."""
    idx = torch.as_tensor(ids, dtype=torch.long)
    return median_seconds(lambda: records.index_select(0, idx), iters)
