"""Pin the slot-table oracle: a hand-worked sequence, brute force against an
independent arg-min formulation, exact-LRU equivalence when every call has one
id, and the reference's own invariants over its recorded router traces."""
import itertools

import numpy as np
import pytest

from oracle import slots


def test_hand_worked_sequence():
    # C = 4: initial stamps -4..-1 make empty slots fill 0, 1, 2, 3 in order;
    # step 3 evicts the lowest-index slot among the two stamped at step 1;
    # step 4 hits expert 1, then evicts the lowest-index slot stamped at step 2.
    tab = slots.SlotTable.fresh(8, 4)
    assert tab.stamp == [-4, -3, -2, -1]
    assert slots.resolve(tab, [0, 1]) == ([0, 1], [0, 1], [0, 1])
    assert slots.resolve(tab, [2, 3]) == ([2, 3], [2, 3], [2, 3])
    assert tab.stamp == [1, 1, 2, 2]
    assert slots.resolve(tab, [4]) == ([0], [0], [4])
    assert tab.slot_of[0] == -1 and tab.slot_expert[0] == 4
    assert slots.resolve(tab, [1, 5]) == ([1, 2], [2], [5])
    assert tab.slot_of[2] == -1 and tab.slot_expert == [4, 1, 5, 3]
    assert tab.stamp == [3, 4, 4, 2] and tab.step == 4
    # a repeated id in one call is a miss then a hit
    assert slots.resolve(tab, [6, 6]) == ([3, 3], [3], [6])


def test_bruteforce_against_lexicographic_argmin():
    E, C, K = 5, 3, 2
    calls = [c for c in itertools.product(range(E), repeat=K) if len(set(c)) == K]
    for seq in itertools.product(calls, repeat=3):
        a = slots.SlotTable.fresh(E, C)
        b = slots.SlotTable.fresh(E, C)
        for ids in seq:
            assert slots.resolve(a, ids) == slots.resolve_lexmin(b, ids)
            assert a.arrays()[0].tolist() == b.arrays()[0].tolist()
            assert a.stamp == b.stamp


def test_single_id_calls_are_exact_lru():
    """With one id per call every stamp is distinct, so the device table is an
    exact LRU and must score the same hits as the OrderedDict simulator
    (bin/simulate_cache.py:64-97)."""
    rng = np.random.default_rng(0)
    recs = [(0, [int(rng.zipf(1.3) % 40)]) for _ in range(3000)]
    for cap in (1, 4, 9, 17):
        assert slots.simulate_slot_table(recs, cap, 40, 1) == slots.simulate(recs, cap, "lru", 1)


@pytest.mark.parametrize("name,cap", [("trace", 64), ("t512", 69), ("direct", 113)])
def test_reference_trace_invariants(traces, name, cap):
    """bin/test_devcache.py:68-72,113-122: every slot handed out holds the
    expert asked for, no slot is handed out twice in a call, tables stay
    mutually inverse, eviction is exercised."""
    layers = traces[f"{name}_decode_layer"]
    ids = traces[f"{name}_decode_ids"]
    tabs = [slots.SlotTable.fresh(256, cap) for _ in range(40)]
    misses = 0
    for layer, row in zip(layers.tolist(), ids.tolist()):
        tab = tabs[layer]
        before = set(e for e in range(256) if tab.slot_of[e] >= 0)
        out, fslot, fexp = slots.resolve(tab, row)
        # every fetch is an id that was absent or was evicted earlier in
        # this same call (only slots touched this step are protected)
        assert set(fexp) <= set(row)
        assert set(row) - before <= set(fexp)
        assert len(set(out)) == len(out)
        assert [tab.slot_expert[s] for s in out] == row
        assert fslot == [out[row.index(e)] for e in fexp]
        misses += len(fexp)
    for tab in tabs:
        so, se, _, _ = tab.arrays()
        for e in range(256):
            if so[e] >= 0:
                assert se[so[e]] == e
        assert sorted(se[se >= 0].tolist()) == sorted(np.flatnonzero(so >= 0).tolist())
    assert misses > 40 * cap                              # eviction happened


def test_host_lru_promised_guard_and_fallback():
    lru = slots.HostLRU(3)
    u, s, c = lru.call([5, 1])
    assert u == [1, 5] and s == [2, 1] and c == [(2, 1), (1, 5)]   # free list pops from the end
    assert lru.call([7, 8, 9, 1]) is None                 # 4 distinct > 3 slots
    u, s, c = lru.call([7])
    assert s == [0]
    # all three slots promised in one call, a fourth expert cannot be placed
    assert lru.call([[1, 5], [7, 2]]) is None


def test_simulator_static_is_an_upper_bound_of_lru_on_reference_trace(traces):
    recs = list(zip(traces["t512_decode_layer"].tolist(), traces["t512_decode_ids"].tolist()))
    for cap in (32, 69, 113):
        lru = slots.simulate(recs, cap, "lru")
        st = slots.simulate(recs, cap, "static")
        dev = slots.simulate_slot_table(recs, cap)
        assert lru[1] == st[1] == dev[1] == len(recs) * 8
        assert st[0] >= lru[0] * 0.9
        assert abs(dev[0] - lru[0]) / lru[1] < 0.02       # step-LRU ~ exact LRU


def test_simulator_static_equals_its_closed_form(traces):
    """Static keeps each layer's `capacity` most frequent experts over the
    whole trace, so its hits are the sum over layers of the top-C counts,
    whatever the order among equal counts (bin/simulate_cache.py:66-71)."""
    import numpy as np
    for name in ("t512", "direct"):
        layer = traces[f"{name}_decode_layer"]
        ids = traces[f"{name}_decode_ids"]
        recs = list(zip(layer.tolist(), ids.tolist()))
        for cap in (1, 8, 32, 69, 113, 256):
            want = 0
            for l in range(40):
                counts = np.bincount(ids[layer == l].ravel(), minlength=256)
                want += int(np.sort(counts)[::-1][:cap].sum())
            assert slots.simulate(recs, cap, "static") == (want, ids.size), (name, cap)


def test_simulator_lfu_hand_worked():
    """LFU evicts the lowest count, and among equal counts the expert
    inserted first (bin/simulate_cache.py:93-94: min over the dict's
    insertion order).  One layer, capacity 3, [1, 2, 3, 4, 1, 2, 3]:
      1 2 3   miss, miss, miss               {1:1, 2:1, 3:1}
      4       miss, evicts 1 (first of the count-1 ties)   {2, 3, 4}
      1       miss, evicts 2                 {3, 4, 1}
      2       miss, evicts 3                 {4, 1, 2}
      3       miss, evicts 4                 {1, 2, 3}
    0 hits; evicting the last-inserted tie would give 2, the lowest id 1.
    Capacity 2, [1, 1, 2, 3, 4, 1]: 1 misses, 1 hits (count 2), 2 misses,
    3 evicts 2 (count 1 < 2), 4 evicts 3, 1 hits: 2 hits, where LRU (which
    evicts 1 at the 3) gets 1."""
    assert slots.simulate([(0, [1, 2, 3, 4, 1, 2, 3])], 3, "lfu") == (0, 7)
    assert slots.simulate([(0, [1, 1, 2, 3, 4, 1])], 2, "lfu") == (2, 6)
    assert slots.simulate([(0, [1, 1, 2, 3, 4, 1])], 2, "lru") == (1, 6)
    # the same calls split over two records and two layers: layers are independent
    assert slots.simulate([(0, [1, 2, 3]), (5, [9]), (0, [4, 1, 2, 3])], 3, "lfu") == (0, 8)
