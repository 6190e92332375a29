"""Known-answer pattern for the expert fetch.

Oracle (test infrastructure).  The reference fills every expert record of its
pinned host region with a self-identifying pattern: element k of expert e,
read as int64, is (e << 32) | k (bin/bench_hostread.py:257-292, pattern at
:284-289), and verifies every fetched byte against it (`Checker`,
:298-327).  The record size is 3,146,496 B = 2^8 * 3 * 17 * 241, so every
record boundary is 256-byte aligned (:84-96).

A fetch is a byte copy: after fetching experts fetch_expert[j] into slots
fetch_slot[j] for j < nmiss, slot fetch_slot[j] holds expert fetch_expert[j]'s
record and every other slot is unchanged (surplus jobs retire without
writing, csrc/fetch_experts.cu:56-60, bin/bench_hostread.py:900-918).
"""
from __future__ import annotations

import numpy as np

EXPERT_BYTES = 3_146_496          # bin/offload.py:603, bin/bench_hostread.py:84
assert EXPERT_BYTES % 256 == 0


def pattern_record(expert: int, record_bytes: int = EXPERT_BYTES) -> np.ndarray:
    """int64 view of one record: (e << 32) | k."""
    n = record_bytes // 8
    return (np.int64(expert) << 32) | np.arange(n, dtype=np.int64)


def which_expert(record_i64: np.ndarray) -> int:
    """Reverse the pattern (bin/bench_hostread.py:321-325)."""
    return int(np.asarray(record_i64)[1] >> 32)


def expected_cache(before: np.ndarray, fetch_expert, fetch_slot, nmiss: int,
                   record_bytes: int = EXPERT_BYTES) -> np.ndarray:
    """int64 [C, record/8] cache contents after a pattern fetch."""
    after = np.array(before, copy=True)
    for j in range(nmiss):
        after[fetch_slot[j]] = pattern_record(fetch_expert[j], record_bytes)
    return after
