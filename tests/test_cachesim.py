"""The product's cache-sizing simulator (cachesim.py) against the oracle's
restatement of bin/simulate_cache.py and of the device table's policy, over
the reference's recorded router traces; the skew report against closed
forms."""
import math

import numpy as np
import pytest

from oracle import slots as oslots


def _records(traces, name):
    return [(int(l), ids.tolist()) for l, ids in zip(traces[f"{name}_decode_layer"],
                                                     traces[f"{name}_decode_ids"])]


@pytest.mark.parametrize("policy", ["lru", "lfu", "static"])
@pytest.mark.parametrize("name,cap", [("trace", 16), ("trace", 64), ("t512", 40),
                                      ("direct", 113)])
def test_policies_equal_the_oracle_on_reference_traces(traces, policy, name, cap):
    import cachesim
    recs = _records(traces, name)
    got = cachesim.policy_hits(recs, cap, policy, 40)
    want = oslots.simulate(recs, cap, policy)
    assert got == want, f"{policy} {name} cap {cap}"


@pytest.mark.parametrize("name,cap", [("trace", 30), ("t512", 69), ("direct", 113)])
def test_step_lru_equals_the_device_table_oracle(traces, name, cap):
    import cachesim
    recs = _records(traces, name)
    assert cachesim.step_lru_hits(recs, cap, 256, 40) == oslots.simulate_slot_table(recs, cap)
    # skipping the first calls counts only the rest
    h, t = cachesim.step_lru_hits(recs, cap, 256, 40, skip=100)
    assert t == 8 * (len(recs) - 100) and 0 < h < t


def test_choose_capacity_is_the_smallest_that_reaches_the_target(traces):
    import cachesim
    recs = _records(traces, "t512")
    cap, rate = cachesim.choose_capacity(recs, 0.6, 256, 40)
    h, t = cachesim.step_lru_hits(recs, cap, 256, 40)
    h1, t1 = cachesim.step_lru_hits(recs, cap - 1, 256, 40)
    assert rate == h / t >= 0.6 > h1 / t1


def test_skew_closed_forms():
    import cachesim
    n = 64
    uniform = [(0, list(range(n)) * 3)]
    r = cachesim.skew(uniform, 2, 256)
    (lay,) = r["layers"]
    assert lay["seen"] == n and lay["entropy"] == pytest.approx(math.log2(n))
    assert lay["gini"] == pytest.approx(0.0, abs=1e-12)
    assert lay["top8_pct"] == pytest.approx(100 * 8 / n)
    # counts 1, 2, ..., n: Gini = (n - 1) / (3 n)
    ramp = [(1, [e for e in range(n) for _ in range(e + 1)])]
    lay = cachesim.skew(ramp, 2, 256)["layers"][0]
    assert lay["layer"] == 1 and lay["gini"] == pytest.approx((n - 1) / (3 * n))
    total = n * (n + 1) / 2
    assert lay["top8_pct"] == pytest.approx(100 * sum(range(n - 7, n + 1)) / total)
    one = cachesim.skew([(0, [5] * 10)], 1, 256)["layers"][0]
    assert one["entropy"] == 0.0 and one["seen"] == 1


def test_skew_of_reference_trace_is_below_uniform(traces):
    import cachesim
    r = cachesim.skew(_records(traces, "t512"), 40, 256)
    assert len(r["layers"]) == 40
    assert 5.0 < r["mean_entropy"] < r["uniform_entropy"] == 8.0
