"""Expert-cache bookkeeping: the device slot table, the host OrderedDict LRU,
and the offline policy simulator.

Oracle (test infrastructure).
"""
from __future__ import annotations

from collections import Counter, OrderedDict
from dataclasses import dataclass, field

import numpy as np


@dataclass
class SlotTable:
    """State of one layer's device cache table (bin/devcache.py:22-24,146-152).

    slot_of[E]      int32  expert -> slot, -1 absent
    slot_expert[C]  int32  slot -> expert, -1 empty
    stamp[C]        int64  step at which the slot was last used
    step            int64  device step counter
    """
    n_experts: int
    cap: int
    slot_of: list = field(default_factory=list)
    slot_expert: list = field(default_factory=list)
    stamp: list = field(default_factory=list)
    step: int = 0

    @classmethod
    def fresh(cls, n_experts: int, cap: int) -> "SlotTable":
        """init_dev_cache (bin/devcache.py:147-152): every slot empty, stamps
        -C..-1 (`-arange(C, 0, -1)`) so the first C misses take slots
        0, 1, 2, ... in order, step 0."""
        return cls(n_experts, cap, [-1] * n_experts, [-1] * cap,
                   [-(cap - c) for c in range(cap)], 0)

    def copy(self) -> "SlotTable":
        return SlotTable(self.n_experts, self.cap, list(self.slot_of),
                         list(self.slot_expert), list(self.stamp), self.step)

    def arrays(self):
        return (np.array(self.slot_of, np.int32), np.array(self.slot_expert, np.int32),
                np.array(self.stamp, np.int64), np.int64(self.step))


def resolve(tab: SlotTable, ids):
    """`_resolve_slots` restated (bin/devcache.py:45-98).  Mutates `tab`.

    step += 1; for each id in order: a hit stamps its slot; a miss evicts
    the slot with the smallest stamp (scan 0..C-1 with strict `<`, so the
    lowest index wins a tie), clears slot_of[victim], installs the id,
    queues (slot, expert) and stamps the slot.  Slots touched this step carry
    the maximum stamp, so none of them can be chosen again in the same call
    (the "promised" guard, bin/devcache.py:77-79).
    Returns (out_slot[K], fetch_slot[nmiss], fetch_expert[nmiss]).
    """
    tab.step += 1
    step = tab.step
    out, fslot, fexp = [], [], []
    for e in ids:
        e = int(e)
        s = tab.slot_of[e]
        if s < 0:
            best = 0
            best_stamp = tab.stamp[0]
            for c in range(1, tab.cap):
                if tab.stamp[c] < best_stamp:
                    best_stamp = tab.stamp[c]
                    best = c
            victim = tab.slot_expert[best]
            if victim >= 0:
                tab.slot_of[victim] = -1
            tab.slot_of[e] = best
            tab.slot_expert[best] = e
            fslot.append(best)
            fexp.append(e)
            s = best
        tab.stamp[s] = step
        out.append(s)
    return out, fslot, fexp


def resolve_lexmin(tab: SlotTable, ids):
    """The same policy written as an arg-min over (stamp, slot) pairs.

    An independent formulation used to cross-check `resolve` by brute force:
    victim = min over slots of the pair (stamp, index).
    """
    tab.step += 1
    out, fslot, fexp = [], [], []
    for e in ids:
        e = int(e)
        s = tab.slot_of[e]
        if s < 0:
            best = min(range(tab.cap), key=lambda c: (tab.stamp[c], c))
            victim = tab.slot_expert[best]
            if victim >= 0:
                tab.slot_of[victim] = -1
            tab.slot_of[e] = best
            tab.slot_expert[best] = e
            fslot.append(best)
            fexp.append(e)
            s = best
        tab.stamp[s] = tab.step
        out.append(s)
    return out, fslot, fexp


class HostLRU:
    """The host-side per-layer cache of `cached_forward` (bin/offload.py:295-317,
    391-451): OrderedDict slot -> expert (oldest first), a free list popped
    from the END, a `promised` set guarding slots already handed out in this
    call, and a fallback (returns None) when the call needs more distinct
    experts than the cache holds or every slot is promised.
    """

    def __init__(self, cap: int):
        self.cap = cap
        self.slot_of: dict[int, int] = {}
        self.lru: OrderedDict[int, int] = OrderedDict()
        self.free = list(range(cap))
        self.hits = 0
        self.misses = 0

    def call(self, ids):
        """ids: all expert ids of the call (any shape).  Returns
        (uniq, slots per uniq, copies [(slot, expert)]) or None on fallback."""
        flat = np.asarray(ids).reshape(-1)
        uniq = sorted(set(int(v) for v in flat))          # torch.unique order
        if len(uniq) > self.cap:
            self.misses += len(uniq)
            return None
        promised: set[int] = set()
        slots, copies = [], []
        for e in uniq:
            slot = self.slot_of.get(e)
            if slot is None:
                self.misses += 1
                if self.free:
                    slot = self.free.pop()
                else:
                    for cand in list(self.lru.keys()):
                        if cand not in promised:
                            victim = self.lru.pop(cand)
                            del self.slot_of[victim]
                            slot = cand
                            break
                    else:
                        return None
                copies.append((slot, e))
                self.slot_of[e] = slot
            else:
                self.hits += 1
            self.lru[slot] = e
            self.lru.move_to_end(slot)
            promised.add(slot)
            slots.append(slot)
        return uniq, slots, copies


def simulate(records, capacity: int, policy: str, layers: int = 40):
    """Offline cache simulation (bin/simulate_cache.py:64-97).

    records: iterable of (layer, ids) where ids is a flat list of expert ids.
    Returns (hits, total).  LRU evicts the least recently used expert one id
    at a time; LFU the lowest count; static keeps the most frequent
    `capacity` experts per layer (an oracle that sees the whole trace).
    """
    records = list(records)
    if policy == "static":
        freq = [Counter() for _ in range(layers)]
        for layer, flat in records:
            freq[layer].update(flat)
        keep = [set(e for e, _ in f.most_common(capacity)) for f in freq]
    caches = [OrderedDict() for _ in range(layers)]
    hits = total = 0
    for layer, flat in records:
        for e in flat:
            total += 1
            if policy == "static":
                hits += e in keep[layer]
                continue
            c = caches[layer]
            if e in c:
                hits += 1
                if policy == "lru":
                    c.move_to_end(e)
                else:
                    c[e] += 1
            else:
                if len(c) >= capacity:
                    if policy == "lru":
                        c.popitem(last=False)
                    else:
                        c.pop(min(c, key=c.get))
                c[e] = 1
    return hits, total


def simulate_slot_table(records, capacity: int, n_experts: int = 256, layers: int = 40):
    """Hit rate of the device slot table itself (step-granular LRU with a
    lowest-slot tie-break) over (layer, ids) records.  Returns (hits, total)."""
    tabs = [SlotTable.fresh(n_experts, capacity) for _ in range(layers)]
    hits = total = 0
    for layer, flat in records:
        _, fslot, _ = resolve(tabs[layer], flat)
        total += len(flat)
        hits += len(flat) - len(fslot)
    return hits, total
