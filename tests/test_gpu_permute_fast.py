"""moe_permute at up to 1024 experts (the 16-wave kernel that places 4096
pairs per pass) against the oracle's stable sort, bit for bit: one expert,
odd expert counts, pair counts that are not a multiple of 64, several
passes, a crowded expert, 32- and 64-bit ids.  Ids outside [0, E) take no
position (pair_pos -1) and are left out of the counts, the order of the
others unchanged: checked against numpy's stable argsort of the valid
pairs."""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import permute as operm

pytestmark = pytest.mark.gpu


def _run(lib, dev, ids_np, E, i32):
    T, K = ids_np.shape
    ids = torch.from_numpy(ids_np).to(dev)
    if i32:
        ids = ids.int()
    mk = lambda n: torch.full((n,), -7, dtype=torch.int32, device=dev)
    counts, offsets, srt, pos = mk(E), mk(E + 1), mk(T * K), mk(T * K)
    lib.permute(ids, E, counts, offsets, srt, pos)
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in (counts, offsets, srt, pos)]


@pytest.mark.parametrize("E,T,K,seed", [(1, 300, 1, 0), (5, 1000, 3, 1), (64, 37, 3, 2),
                                        (256, 512, 8, 3), (256, 700, 8, 4), (1024, 1125, 8, 5),
                                        (1000, 4096, 4, 6), (300, 2048, 8, 7)])
def test_permute_up_to_1024_experts(lib, dev, E, T, K, seed):
    rng = np.random.default_rng(seed)
    ids_np = rng.integers(0, E, (T, K))
    if E >= 300:
        ids_np[: min(T, 300), 0] = E - 1                # one crowded expert
    for i32 in (False, True):
        say(f"permute fast: E={E} T={T} K={K} ({T * K} pairs, {'int32' if i32 else 'int64'})")
        got = _run(lib, dev, ids_np, E, i32)
        want = operm.permute(ids_np, E)
        for g, w, name in zip(got, want, ("counts", "offsets", "sorted_pairs", "pair_pos")):
            assert np.array_equal(g, w), name


def test_permute_out_of_range_ids(lib, dev):
    E, T, K = 64, 200, 8
    rng = np.random.default_rng(9)
    ids_np = rng.integers(0, E, (T, K))
    bad = rng.random((T, K)) < 0.05
    ids_np[bad] = rng.choice([-3, -1, E, E + 5, 1 << 20], size=int(bad.sum()))
    say("permute fast: out-of-range ids")
    counts, offsets, srt, pos = _run(lib, dev, ids_np, E, i32=False)
    flat = ids_np.reshape(-1)
    valid = (flat >= 0) & (flat < E)
    idx = np.nonzero(valid)[0]
    want_sorted = idx[np.argsort(flat[idx], kind="stable")]
    n = idx.size
    assert np.array_equal(counts, np.bincount(flat[valid], minlength=E))
    assert offsets[E] == n and np.array_equal(offsets[:E], np.cumsum(counts) - counts)
    assert np.array_equal(srt[:n], want_sorted)
    want_pos = np.full(flat.size, -1)
    want_pos[want_sorted] = np.arange(n)
    assert np.array_equal(pos, want_pos)
