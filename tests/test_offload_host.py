"""Host logic of the offload hooks (bin/offload.py), on the CPU: the
host-managed cache's slot and copy decisions against the oracle's restatement
of cached_forward over the reference's recorded router traces, the counters,
the census and the router trace."""
import json

import numpy as np
import pytest
import torch

from oracle import slots as oslots


def _decode_calls(traces, name):
    return zip(traces[f"{name}_decode_layer"].tolist(), traces[f"{name}_decode_ids"])


def _prefill_calls(traces):
    rows, ids = traces["trace_prefill_rows"], traces["trace_prefill_ids"]
    at = 0
    for layer, n in zip(traces["trace_prefill_layer"].tolist(), rows.tolist()):
        yield layer, ids[at:at + n]
        at += n


@pytest.mark.parametrize("name,cap", [("trace", 8), ("trace", 64), ("t512", 113),
                                      ("direct", 30), ("direct", 200)])
def test_host_lru_decisions_equal_the_oracle_on_reference_traces(traces, name, cap):
    """Per layer: the same slot for every distinct expert, the same
    (slot, expert) copies in the same order, the same fallbacks, and the
    same hit/miss counts as oracle.slots.HostLRU (cached_forward restated),
    call after call over a recorded trace -- prefill calls (up to 512 rows)
    first when the trace has them, then every decode call."""
    import offload
    calls = list(_prefill_calls(traces)) if name == "trace" else []
    calls += list(_decode_calls(traces, name))
    ours = [offload._HostLRU(cap, 256) for _ in range(40)]
    want = [oslots.HostLRU(cap) for _ in range(40)]
    hits = misses = fallbacks = 0
    for i, (layer, ids) in enumerate(calls):
        uniq = np.unique(np.asarray(ids).reshape(-1))
        got = ours[layer].plan(uniq)
        exp = want[layer].call(ids)
        if exp is None:
            assert got is None, f"call {i}: the oracle falls back"
            fallbacks += 1
            continue
        assert got is not None, f"call {i}: unexpected fallback"
        slots, copies, h, m = got
        assert [int(u) for u in exp[0]] == uniq.tolist()
        assert slots == exp[1], f"call {i} (layer {layer}): slots"
        assert copies == exp[2], f"call {i} (layer {layer}): copies"
        hits += h
        misses += m
    assert hits == sum(w.hits for w in want)
    assert misses == sum(w.misses for w in want) - sum(
        len(np.unique(np.asarray(ids))) for l, ids in calls
        if len(np.unique(np.asarray(ids))) > cap)
    print(f"{name} cap {cap}: {len(calls)} calls, hits {hits}, misses {misses}, "
          f"fallbacks {fallbacks}")
    if cap < 64 and name == "trace":
        assert fallbacks > 0                                  # the n > cap path is exercised
    assert misses > cap                                       # eviction is exercised


def test_host_lru_hand_worked():
    """C = 3.  Unused slots go out from the top (2, 1, 0); then the least
    recently used slot not taken by this call is evicted."""
    import offload
    lru = offload._HostLRU(3, 10)
    assert lru.plan([4, 7]) == ([2, 1], [(2, 4), (1, 7)], 0, 2)
    assert lru.plan([1, 7]) == ([0, 1], [(0, 1)], 1, 1)
    # 4 (slot 2) is the least recently used; 7 and 1 were used later
    assert lru.plan([5]) == ([2], [(2, 5)], 0, 1)
    # this call takes slot 0 (expert 1, a hit) first; the miss of 8 must not
    # evict it even though slot 1 (expert 7) is older
    assert lru.plan([1, 8]) == ([0, 1], [(1, 8)], 1, 1)
    assert lru.plan([0, 1, 2, 3]) is None                     # more experts than slots


def test_stats_fold_device_tallies_on_read():
    import offload
    st = offload._Stats(experts_copied=0, bytes_copied=0, hits=0, misses=0, gather_hits=0,
                        gather_misses=0)
    tally = torch.zeros(2, dtype=torch.int64)
    st.watch(tally, 1000)
    st.watch(tally, 1000)                                     # watched once
    st.add(hits=3, misses=2)
    tally += torch.tensor([4, 5])
    assert st["gather_hits"] == 4 and st["gather_misses"] == 5
    assert st["experts_copied"] == 9 and st["bytes_copied"] == 9000
    tally += torch.tensor([1, 0])
    assert dict(st.items())["gather_hits"] == 5 and st["experts_copied"] == 10
    assert st["hits"] == 3 and st["misses"] == 2


def test_router_trace_and_census(tmp_path):
    import offload
    offload.enable_census(2, 8)
    offload.TRACE.enabled = True
    offload.TRACE.clear()
    try:
        assert offload.CENSUS.shape == (2, 8)
        offload._count(1, torch.tensor([[1, 2, 3]]))
        offload._count(1, torch.tensor([[1, 2, 3], [3, 4, 5]]))
        offload._count(-1, torch.tensor([[0, 0, 0]]))              # no layer index: ignored
        offload.TRACE.add(1, torch.tensor([[1, 2, 3]]))
        offload.TRACE.add(0, torch.tensor([[1, 2], [3, 4]]))
        assert offload.CENSUS[1].tolist() == [0, 2, 2, 3, 1, 1, 0, 0]
        assert offload.CENSUS_DECODE[1].tolist() == [0, 1, 1, 1, 0, 0, 0, 0]
        assert offload.CENSUS[0].tolist() == [0] * 8
        offload._count(1, torch.tensor([[7, 7, 6]]))
        assert offload.CENSUS[1].tolist() == [0, 2, 2, 3, 1, 1, 1, 2]
        offload._count(1, torch.tensor([[8, -1, 6]]))               # ids outside the census: dropped
        assert offload.CENSUS[1].tolist() == [0, 2, 2, 3, 1, 1, 2, 2]
        recs = offload.TRACE.records
        assert [r["phase"] for r in recs] == ["decode", "prefill"]
        assert recs[1] == {"phase": "prefill", "layer": 0, "ids": [[1, 2], [3, 4]]}
        assert offload.TRACE.first_decode is not None
        out = tmp_path / "trace.json"
        offload.TRACE.save(out, {"frames": 1})
        saved = json.loads(out.read_text())
        assert saved["meta"] == {"frames": 1} and saved["records"] == recs
    finally:
        offload.disable_census()
        offload.TRACE.enabled = False
        offload.TRACE.clear()
    assert offload.CENSUS is None and offload.CENSUS_DECODE is None


def test_memory_snapshot_keys():
    import offload
    snap = offload.memory_snapshot(None)
    assert snap["ram_peak_gib"] > 0 and "ram_rss_gib" in snap


def test_host_arena_layout():
    """The four buffers of a layer in one allocation, each 256-byte aligned,
    values kept when re-homed."""
    import moe
    import offload
    m = moe.MoEExperts(4, 256, 128)
    m.w13_scale_inv.copy_(torch.arange(m.w13_scale_inv.numel()).view_as(m.w13_scale_inv))
    offload._to_host_arena(m, pinned=False, keep_values=True)
    bases = [getattr(m, n).data_ptr() for n in offload._BUFFERS]
    assert all(b % 256 == 0 for b in bases)
    assert bases == sorted(bases) and bases[-1] - bases[0] < m._host_arena.nbytes
    assert m.w13_scale_inv.flatten().tolist() == list(range(m.w13_scale_inv.numel()))
    assert sorted(n for n, _ in m.named_buffers()) == sorted(offload._BUFFERS)


class _StandInLib:
    """host_alloc/host_free over memory this test owns, for Native.host_buffer
    on the CPU: records what is freed, and when."""

    def __init__(self):
        import ctypes
        self.blocks, self.freed = {}, []
        self._ctypes = ctypes

    def host_alloc(self, nbytes, noncoherent=False):
        b = self._ctypes.create_string_buffer(nbytes + 256)
        ptr = (self._ctypes.addressof(b) + 255) // 256 * 256
        self.blocks[ptr] = b
        return ptr

    def host_free(self, ptr):
        self.freed.append(ptr)
        del self.blocks[ptr]


def test_host_buffer_lives_as_long_as_its_views():
    """Page-locked memory handed out by host_buffer is freed only when its
    last view is gone (a slice of a pool outliving the pool, the module's
    buffers outliving the arena object), after the range hooks; nothing is
    freed at interpreter exit."""
    import gc
    import hipfetch
    fake = _StandInLib()
    seen = []
    ptr, arr = hipfetch.Native.host_buffer(fake, 4096, on_free=(lambda lo, hi: seen.append((lo, hi)),))
    t = torch.from_numpy(arr.reshape(4, 1024))
    part = t[2:].view(torch.int32)
    part.fill_(7)
    del arr, t
    gc.collect()
    assert fake.freed == [] and seen == []
    assert int(part.sum()) == 7 * 512              # the memory is still there
    del part
    gc.collect()
    assert fake.freed == [ptr] and seen == [(ptr, ptr + 4096)]
    # at exit: the finaliser is not one weakref runs then
    _, keep = hipfetch.Native.host_buffer(fake, 256)
    import weakref
    ours = [f for f in list(weakref.finalize._registry)
            if f.alive and f.peek()[1] is hipfetch._free_host_buffer]
    assert len(ours) == 1 and not ours[0].atexit
    del keep
    gc.collect()
