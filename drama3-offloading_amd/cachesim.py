"""Offline cache sizing: how skewed the routing is, and how a per-layer expert
cache of a given capacity would do on an expert-id stream, without a GPU.

Counterpart of bin/simulate_cache.py: the skew report (:31-61), the LRU /
LFU / static policy replay (:64-97), plus the step-granular LRU that the
device slot table actually implements (bin/devcache.py:65-98), used to size
the decode cache.  Records are (layer, ids) pairs, ids any iterable of
expert ids (a decode call's 8, or a prefill call's rows flattened).

Each policy keeps its state in per-layer arrays indexed by expert id:
  lru     last-use time; a miss on a full cache evicts the resident expert
          used longest ago;
  lfu     hit count since insertion (1 on insertion) and insertion time; a
          miss evicts the lowest count, the earliest inserted on a tie;
  static  the `capacity` most frequent experts of the whole stream per layer
          (ties to the expert seen first), fixed in advance -- a bound that
          sees the future.
"""
from __future__ import annotations

import math

import numpy as np


def _flat(ids) -> list[int]:
    return np.asarray(ids, dtype=np.int64).reshape(-1).tolist()


def skew(records, layers: int, n_experts: int) -> dict:
    """Per-layer routing skew: experts seen, entropy of the id distribution
    (bits; uniform over 256 is 8), Gini coefficient (0 uniform, -> 1 one
    expert), and the share of calls taken by the 8 and 32 most used experts
    (bin/simulate_cache.py:31-61).  Returns {"layers": [...], "mean_entropy":
    bits over the layers that saw any id}."""
    counts = np.zeros((layers, n_experts), np.int64)
    for layer, ids in records:
        np.add.at(counts[layer], np.asarray(_flat(ids), np.int64), 1)
    out = []
    for layer in range(layers):
        c = counts[layer][counts[layer] > 0]
        if c.size == 0:
            continue
        p = c / c.sum()
        desc = np.sort(c)[::-1]
        asc = desc[::-1]
        n = c.size
        # Gini of the seen experts' counts: 2 sum_i i x_(i) / (n sum x) - (n + 1) / n
        gini = 2.0 * float(np.dot(np.arange(1, n + 1), asc)) / (n * c.sum()) - (n + 1) / n
        out.append({"layer": layer, "seen": int(n),
                    "entropy": float(-(p * np.log2(p)).sum()),
                    "gini": float(gini),
                    "top8_pct": float(100.0 * desc[:8].sum() / c.sum()),
                    "top32_pct": float(100.0 * desc[:32].sum() / c.sum())})
    ents = [r["entropy"] for r in out]
    return {"layers": out, "mean_entropy": float(np.mean(ents)) if ents else 0.0,
            "uniform_entropy": math.log2(n_experts)}


def policy_hits(records, capacity: int, policy: str, layers: int,
                n_experts: int = 256) -> tuple[int, int]:
    """Replay `records` one id at a time against a per-layer cache of
    `capacity` experts under `policy` ("lru", "lfu" or "static").  Returns
    (hits, total)."""
    records = list(records)
    if policy == "static":
        return _static_hits(records, capacity, layers, n_experts)
    if policy not in ("lru", "lfu"):
        raise ValueError(f"unknown policy {policy!r}")
    resident = np.zeros((layers, n_experts), bool)
    size = np.zeros(layers, np.int64)
    stamp = np.zeros((layers, n_experts), np.int64)     # lru: last use; lfu: insertion time
    hits_of = np.zeros((layers, n_experts), np.int64)   # lfu only
    big = np.iinfo(np.int64).max
    clock = hits = total = 0
    for layer, ids in records:
        res, st, hc = resident[layer], stamp[layer], hits_of[layer]
        for e in _flat(ids):
            clock += 1
            total += 1
            if res[e]:
                hits += 1
                if policy == "lru":
                    st[e] = clock
                else:
                    hc[e] += 1
                continue
            if size[layer] >= capacity:
                if policy == "lru":
                    victim = int(np.where(res, st, big).argmin())
                else:
                    # lowest count, then earliest insertion: one key per expert
                    key = np.where(res, hc * (clock + 1) + st, big)
                    victim = int(key.argmin())
                res[victim] = False
                size[layer] -= 1
            res[e] = True
            size[layer] += 1
            st[e] = clock
            hc[e] = 1
    return hits, total


def _static_hits(records, capacity, layers, n_experts):
    counts = np.zeros((layers, n_experts), np.int64)
    first = np.full((layers, n_experts), np.iinfo(np.int64).max, np.int64)
    at = 0
    for layer, ids in records:
        for e in _flat(ids):
            counts[layer, e] += 1
            first[layer, e] = min(first[layer, e], at)
            at += 1
    keep = np.zeros((layers, n_experts), bool)
    for layer in range(layers):
        seen = np.nonzero(counts[layer])[0]
        order = sorted(seen.tolist(), key=lambda e: (-counts[layer, e], first[layer, e]))
        keep[layer, order[:capacity]] = True
    hits = total = 0
    for layer, ids in records:
        f = _flat(ids)
        total += len(f)
        hits += int(keep[layer, f].sum())
    return hits, total


def lru_hits(records, capacity: int, layers: int, n_experts: int = 256) -> tuple[int, int]:
    """Exact per-id LRU (bin/simulate_cache.py:64-97's "lru")."""
    return policy_hits(records, capacity, "lru", layers, n_experts)


def step_lru_hits(records, capacity: int, n_experts: int, layers: int,
                  skip: int = 0) -> tuple[int, int]:
    """The device slot table's policy: every id of a call is stamped with the
    call's step; a miss takes the slot with the smallest stamp, the lowest
    slot on a tie, with initial stamps -C..-1 so empty slots fill in order.
    Calls before `skip` warm the cache without being counted.  Returns
    (hits, total)."""
    slot_of = np.full((layers, n_experts), -1, np.int64)
    owner = np.full((layers, capacity), -1, np.int64)
    stamp = np.tile(np.arange(-capacity, 0, dtype=np.int64), (layers, 1))
    step = np.zeros(layers, np.int64)
    hits = total = 0
    for i, (layer, ids) in enumerate(records):
        step[layer] += 1
        so, ow, st = slot_of[layer], owner[layer], stamp[layer]
        counted = i >= skip
        for e in _flat(ids):
            s = so[e]
            if s < 0:
                s = int(st.argmin())                     # argmin takes the first minimum
                if ow[s] >= 0:
                    so[ow[s]] = -1
                so[e] = s
                ow[s] = e
            elif counted:
                hits += 1
            st[s] = step[layer]
            total += counted
    return hits, total


def choose_capacity(records, target: float, n_experts: int, layers: int, skip: int = 0,
                    lo: int = 8, hi: int | None = None) -> tuple[int, float]:
    """Smallest capacity in [lo, hi] whose step-LRU hit rate reaches `target`
    (bisection: the rate does not fall as capacity grows).  Returns
    (capacity, its hit rate); hi and its rate when even hi falls short."""
    hi = n_experts if hi is None else hi
    records = list(records)

    def rate(c):
        h, t = step_lru_hits(records, c, n_experts, layers, skip)
        return h / t if t else 0.0

    if rate(hi) < target:
        return hi, rate(hi)
    while lo < hi:
        mid = (lo + hi) // 2
        if rate(mid) >= target:
            hi = mid
        else:
            lo = mid + 1
    return lo, rate(lo)
