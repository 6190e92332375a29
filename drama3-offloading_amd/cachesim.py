"""Offline cache sizing: replay expert-id streams against an LRU and pick the
capacity that reaches a target hit rate.

Counterpart of bin/simulate_cache.py (policy simulation over a router trace,
:64-97) plus the step-granular variant that the device slot table actually
implements, used to size the per-layer cache of the decode harness.
"""
from __future__ import annotations

from collections import OrderedDict


def lru_hits(records, capacity: int, layers: int) -> tuple[int, int]:
    """records: iterable of (layer, ids).  Exact LRU per layer, one id at a
    time (bin/simulate_cache.py:73-97).  Returns (hits, total)."""
    caches = [OrderedDict() for _ in range(layers)]
    hits = total = 0
    for layer, ids in records:
        c = caches[layer]
        for e in ids:
            total += 1
            if e in c:
                hits += 1
                c.move_to_end(e)
            else:
                if len(c) >= capacity:
                    c.popitem(last=False)
                c[e] = True
    return hits, total


def step_lru_hits(records, capacity: int, n_experts: int, layers: int,
                  skip: int = 0) -> tuple[int, int]:
    """The device table's policy (stamp = step, evict the smallest stamp,
    lowest slot on a tie, initial stamps -C..-1).  Calls before `skip`
    warm the cache without being counted.  Returns (hits, total)."""
    slot_of = [[-1] * n_experts for _ in range(layers)]
    slot_exp = [[-1] * capacity for _ in range(layers)]
    stamp = [[-(capacity - c) for c in range(capacity)] for _ in range(layers)]
    step = [0] * layers
    hits = total = 0
    for i, (layer, ids) in enumerate(records):
        step[layer] += 1
        so, se, st = slot_of[layer], slot_exp[layer], stamp[layer]
        for e in ids:
            s = so[e]
            if s < 0:
                s = min(range(capacity), key=st.__getitem__)   # first minimum
                v = se[s]
                if v >= 0:
                    so[v] = -1
                so[e] = s
                se[s] = e
            elif i >= skip:
                hits += 1
            st[s] = step[layer]
            if i >= skip:
                total += 1
    return hits, total


def choose_capacity(records, target: float, n_experts: int, layers: int, skip: int = 0,
                    lo: int = 8, hi: int | None = None) -> tuple[int, float]:
    """Smallest capacity in [lo, hi] whose step-LRU hit rate >= target
    (binary search; the hit rate is monotone in capacity for LRU)."""
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
