"""Pin the permute/unique/unpermute and fetch-pattern oracles."""
import numpy as np
import torch

from oracle import fetch, permute


def test_permute_matches_bruteforce_on_reference_prefill(traces):
    rows = traces["trace_prefill_rows"]
    ids = traces["trace_prefill_ids"]
    start = 0
    for r in rows[:6]:
        blk = ids[start:start + r].astype(np.int64)
        start += r
        a = permute.permute(blk, 256)
        b = permute.permute_bruteforce(blk, 256)
        for x, y in zip(a, b):
            assert np.array_equal(x, y)
        counts, offsets, sp, pos = a
        flat = blk.reshape(-1)
        assert np.all(np.diff(flat[sp]) >= 0)                       # grouped by expert
        assert np.array_equal(sp[pos], np.arange(flat.size))         # inverse


def test_unique_inverse_matches_torch_unique(traces):
    blk = traces["trace_prefill_ids"][:55].astype(np.int64)
    u, inv = permute.unique_inverse(blk)
    tu, tinv = torch.unique(torch.from_numpy(blk).reshape(-1), return_inverse=True)
    assert np.array_equal(u, tu.numpy())
    assert np.array_equal(inv.reshape(-1), tinv.numpy())
    assert np.array_equal(u[inv], blk)


def test_unpermute_closed_form():
    ids = np.array([[2, 0], [0, 1]])
    _, _, sp, pos = permute.permute(ids, 3)
    H = 4
    y = np.zeros((4, H))
    for p in range(4):                     # row for pair p at its permuted position
        y[pos[p]] = p + 1
    w = np.array([[0.5, 0.25], [2.0, 1.0]])
    out = permute.unpermute(y, pos, w, 2)
    assert np.array_equal(out[:, 0], [0.5 * 1 + 0.25 * 2, 2.0 * 3 + 1.0 * 4])


def test_fetch_pattern_and_expected_cache():
    rec = fetch.pattern_record(7, 4096)
    assert rec[0] == 7 << 32 and rec[5] == (7 << 32) | 5
    assert fetch.which_expert(rec) == 7
    before = np.full((4, 512), -1, np.int64)
    after = fetch.expected_cache(before, [9, 3, 5], [2, 0, 1], 2, 4096)
    assert fetch.which_expert(after[2]) == 9 and fetch.which_expert(after[0]) == 3
    assert np.all(after[1] == -1) and np.all(after[3] == -1)     # surplus job retired
    assert fetch.EXPERT_BYTES == 2 * 512 * 2048 + 2048 * 512 + 8 * 16 * 4 + 16 * 4 * 4


def test_gather_plan_reads_the_table_only_and_covers_every_expert():
    """Every distinct expert lands in exactly one list at its own gather row;
    resident ones name their slot; the table is unchanged."""
    from oracle import permute as op
    rng = np.random.default_rng(4)
    E, C = 256, 40
    slot_of = np.full(E, -1, np.int32)
    resident = rng.choice(E, C, replace=False)
    slot_of[resident] = rng.permutation(C)
    before = slot_of.copy()
    uniq = np.unique(rng.integers(0, E, 300))
    he, hd, cs, cd = op.gather_plan(uniq, slot_of, C)
    assert np.array_equal(slot_of, before)
    assert sorted(np.concatenate([hd, cd]).tolist()) == list(range(uniq.size))
    assert all(slot_of[uniq[d]] == s for s, d in zip(cs, cd))
    assert all(slot_of[e] < 0 and uniq[d] == e for e, d in zip(he, hd))
    assert cs.size == np.isin(uniq, resident).sum()
    he0, hd0, cs0, _ = op.gather_plan(uniq, None, 0)
    assert np.array_equal(he0, uniq) and cs0.size == 0
