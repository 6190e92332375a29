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
