"""Token -> expert permutation and its inverse.

Oracle (test infrastructure).

* `unique_inverse` is the reference's own remap: `torch.unique(ids.cpu(),
  return_inverse=True)` gives the sorted distinct experts and, for every
  (token, k) pair, its index into that list; the expert weights are then
  gathered in that order and the kernel receives the renumbered ids
  (bin/offload.py:157-158, 409, 447-448).
* `permute` is the grouping a grouped GEMM needs: pairs sorted by expert,
  stable in pair order (pair p = t*K + k).  Upstream's fp8_moe_forward does
  this sort internally (not visible in the reference); the stable order is
  this build's contract, and because every row is computed independently and
  `unpermute` sums over k in a fixed order, outputs do not depend on it.
* `unpermute`: out[t] = sum_k w[t,k] * y[pos[t*K+k]] in k order.
"""
from __future__ import annotations

import numpy as np


def unique_inverse(ids):
    flat = np.asarray(ids, np.int64).reshape(-1)
    uniq, inv = np.unique(flat, return_inverse=True)
    return uniq, inv.reshape(np.asarray(ids).shape)


def permute(ids, n_experts: int):
    """ids [T, K] -> (counts[E], offsets[E+1], sorted_pairs[T*K], pair_pos[T*K])."""
    flat = np.asarray(ids, np.int64).reshape(-1)
    counts = np.bincount(flat, minlength=n_experts).astype(np.int32)
    offsets = np.zeros(n_experts + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    sorted_pairs = np.argsort(flat, kind="stable").astype(np.int32)
    pair_pos = np.empty_like(sorted_pairs)
    pair_pos[sorted_pairs] = np.arange(flat.size, dtype=np.int32)
    return counts, offsets, sorted_pairs, pair_pos


def permute_bruteforce(ids, n_experts: int):
    """Same result by a direct double loop (cross-check of `permute`)."""
    flat = [int(v) for v in np.asarray(ids).reshape(-1)]
    counts = [0] * n_experts
    for e in flat:
        counts[e] += 1
    offsets = [0]
    for c in counts:
        offsets.append(offsets[-1] + c)
    sorted_pairs = []
    for e in range(n_experts):
        for p, v in enumerate(flat):
            if v == e:
                sorted_pairs.append(p)
    pair_pos = [0] * len(flat)
    for pos, p in enumerate(sorted_pairs):
        pair_pos[p] = pos
    return (np.array(counts, np.int32), np.array(offsets, np.int32),
            np.array(sorted_pairs, np.int32), np.array(pair_pos, np.int32))


def unpermute(y_perm, pair_pos, weights, top_k: int):
    """y_perm [P, H], pair_pos [T*K], weights [T, K] -> float64 [T, H]."""
    y = np.asarray(y_perm, np.float64)
    w = np.asarray(weights, np.float64)
    T = w.shape[0]
    pos = np.asarray(pair_pos).reshape(T, top_k)
    out = np.zeros((T, y.shape[1]), np.float64)
    for k in range(top_k):
        out += w[:, k:k + 1] * y[pos[:, k]]
    return out


def gather_plan(uniq, slot_of, cap: int):
    """Hybrid prefill gather (bin/offload.py:195-224): for i, e in
    enumerate(uniq), a resident expert (slot_of[e] >= 0, i.e. in [0, cap))
    is copied from its cache slot into gather row i, any other expert from
    its host record.  Returns (host_expert, host_dst, cache_src, cache_dst),
    each in uniq order; the table is not modified."""
    host_e, host_d, cache_s, cache_d = [], [], [], []
    for i, e in enumerate(int(v) for v in np.asarray(uniq).reshape(-1)):
        s = int(slot_of[e]) if slot_of is not None else -1
        if 0 <= s < cap:
            cache_s.append(s)
            cache_d.append(i)
        else:
            host_e.append(e)
            host_d.append(i)
    as32 = lambda v: np.array(v, np.int32)      # noqa: E731
    return as32(host_e), as32(host_d), as32(cache_s), as32(cache_d)
