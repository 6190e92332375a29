"""Expert fetch on the GPU: byte-exact against the self-identifying pattern
(bin/bench_hostread.py:257-327), surplus jobs retire, DYNAMIC under graph
replay (bin/bench_hostread.py:852-934)."""
import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu
RB = 3_146_496
W64 = RB // 8


@pytest.fixture(scope="module")
def pool():
    """256 pinned records carrying (e << 32) | k."""
    n = 256
    say("fetch: building 256-record pinned pattern pool")
    host = torch.empty(n * RB, dtype=torch.uint8, pin_memory=True)
    h64 = host.view(torch.int64).view(n, W64)
    k = torch.arange(W64, dtype=torch.int64)
    for e in range(n):
        torch.add(k, e << 32, out=h64[e])
    return host


def _check(cache, ids, slot0=0):
    d64 = cache.view(torch.int64).view(cache.shape[0] // RB, W64)
    k = torch.arange(W64, dtype=torch.int64, device=cache.device)
    bad = 0
    for j, e in enumerate(ids):
        bad += int((d64[slot0 + j] != k + (int(e) << 32)).sum())
    return bad


def _untouched(cache, lo, hi):
    d64 = cache.view(torch.int64).view(cache.shape[0] // RB, W64)
    return bool((d64[lo:hi] == -1).all())


@pytest.mark.parametrize("length", [8, 32, 64, 128])
def test_fetch_zipf_lists_byte_exact(lib, dev, pool, length):
    rng = np.random.default_rng(20261017 + length)
    import synth
    ids = synth.zipf_miss_list(rng, length)
    cache = torch.full((128 * RB,), 255, dtype=torch.uint8, device=dev)
    fexp = torch.tensor(ids, dtype=torch.int32, device=dev)
    fslot = torch.arange(length, dtype=torch.int32, device=dev)
    nmiss = torch.tensor([length], dtype=torch.int32, device=dev)
    src = lib.device_ptr_of(pool.data_ptr())
    say(f"fetch: zipf list of {length}")
    lib.fetch([(src, cache.data_ptr(), RB)], fexp, fslot, nmiss, max_jobs=length,
              blocks_per_job=64)
    torch.cuda.synchronize()
    assert _check(cache, ids) == 0
    assert _untouched(cache, length, 128)


def test_fetch_list_of_256_as_two_replays_of_128(lib, dev, pool):
    """A 256-long miss list exceeds the 128-slot cache: it runs as two
    128-job launches over the two halves of the list, each checked."""
    import synth
    ids = synth.zipf_miss_list(np.random.default_rng(20261273), 256)
    cache = torch.full((128 * RB,), 255, dtype=torch.uint8, device=dev)
    fslot = torch.arange(128, dtype=torch.int32, device=dev)
    nmiss = torch.tensor([128], dtype=torch.int32, device=dev)
    src = lib.device_ptr_of(pool.data_ptr())
    say("fetch: zipf list of 256 as 2 x 128")
    for half in (ids[:128], ids[128:]):
        fexp = torch.tensor(half, dtype=torch.int32, device=dev)
        lib.fetch([(src, cache.data_ptr(), RB)], fexp, fslot, nmiss, max_jobs=128,
                  blocks_per_job=2)
        torch.cuda.synchronize()
        assert _check(cache, half) == 0


def test_fetch_honours_device_side_job_count(lib, dev, pool):
    cache = torch.full((8 * RB,), 255, dtype=torch.uint8, device=dev)
    ids = [200, 3, 77, 150, 9, 1, 255, 64]
    fexp = torch.tensor(ids, dtype=torch.int32, device=dev)
    fslot = torch.tensor([7, 6, 5, 4, 3, 2, 1, 0], dtype=torch.int32, device=dev)
    nmiss = torch.tensor([3], dtype=torch.int32, device=dev)
    src = lib.device_ptr_of(pool.data_ptr())
    say("fetch: nmiss 3 of a grid of 8")
    lib.fetch([(src, cache.data_ptr(), RB)], fexp, fslot, nmiss, max_jobs=8, blocks_per_job=16)
    torch.cuda.synchronize()
    d64 = cache.view(torch.int64).view(8, W64)
    assert int(d64[7, 1] >> 32) == 200 and int(d64[6, 1] >> 32) == 3 and int(d64[5, 1] >> 32) == 77
    assert _untouched(cache, 0, 5)


def test_fetch_four_pairs_including_unaligned(lib, dev):
    """The four reference buffers in one launch, plus an 8-byte-per-record
    pair (the toy-shape case the reference routed to Triton,
    bin/devcache.py:205-212)."""
    n, C = 16, 6
    sizes = [4096, 2048, 48, 8]
    hosts, caches, pairs = [], [], []
    for i, b in enumerate(sizes):
        h = torch.empty(n * b, dtype=torch.uint8, pin_memory=True)
        h.copy_(torch.randint(0, 256, (n * b,), dtype=torch.uint8))
        c = torch.zeros(C * b, dtype=torch.uint8, device=dev)
        hosts.append(h)
        caches.append(c)
        pairs.append((lib.device_ptr_of(h.data_ptr()), c.data_ptr(), b))
    fexp = torch.tensor([5, 0, 15, 9], dtype=torch.int32, device=dev)
    fslot = torch.tensor([2, 5, 0, 3], dtype=torch.int32, device=dev)
    nmiss = torch.tensor([4], dtype=torch.int32, device=dev)
    say("fetch: four pairs incl. 8-byte records")
    lib.fetch(pairs, fexp, fslot, nmiss, max_jobs=4, blocks_per_job=3)
    torch.cuda.synchronize()
    for h, c, b in zip(hosts, caches, sizes):
        hv, cv = h.view(n, b), c.cpu().view(C, b)
        for e, s in zip([5, 0, 15, 9], [2, 5, 0, 3]):
            assert torch.equal(cv[s], hv[e])
        assert torch.all(cv[1] == 0) and torch.all(cv[4] == 0)


def test_fetch_tile_order_pairs(lib, dev):
    """tile_k = K: each row-major [R, K] host matrix lands in MFMA tile
    order (hostpool.to_tiles), beside a byte pair in the same launch.
    Shapes: the Drama-3 w13 [1024, 2048] and w2 [2048, 512], K = 384 with
    1.5 pieces of 8 KiB per record (a partial piece), and one 16 x 128 tile
    (less than a piece)."""
    from hostpool import to_tiles
    n, C = 12, 5
    mats = [(1024, 2048), (2048, 512), (32, 384), (16, 128)]
    g = torch.Generator().manual_seed(3)
    ids, slots = [7, 0, 11, 4], [3, 0, 4, 1]
    fexp = torch.tensor(ids, dtype=torch.int32, device=dev)
    fslot = torch.tensor(slots, dtype=torch.int32, device=dev)
    nmiss = torch.tensor([len(ids)], dtype=torch.int32, device=dev)
    for first, second in ((0, 1), (2, 3)):
        hosts, caches, pairs = [], [], []
        for R, Kd in (mats[first], mats[second]):
            h = torch.randint(0, 256, (n, R, Kd), dtype=torch.uint8, generator=g).pin_memory()
            c = torch.zeros((C, R, Kd), dtype=torch.uint8, device=dev)
            hosts.append(h)
            caches.append(c)
            pairs.append((lib.device_ptr_of(h.data_ptr()), c.data_ptr(), R * Kd, Kd))
        hs = torch.randint(0, 256, (n, 48), dtype=torch.uint8, generator=g).pin_memory()
        cs = torch.zeros((C, 48), dtype=torch.uint8, device=dev)
        pairs.append((lib.device_ptr_of(hs.data_ptr()), cs.data_ptr(), 48, 0))
        say(f"fetch: tile order {mats[first]} {mats[second]} + 48-byte pair")
        lib.fetch(pairs, fexp, fslot, nmiss, max_jobs=4, blocks_per_job=3)
        torch.cuda.synchronize()
        for h, c in zip(hosts, caches):
            got = c.cpu()
            for e, s_ in zip(ids, slots):
                assert torch.equal(got[s_], to_tiles(h[e])), (tuple(h.shape[1:]), e)
            assert torch.all(got[2] == 0)
        for e, s_ in zip(ids, slots):
            assert torch.equal(cs[s_].cpu(), hs[e])


def test_fetch_tile_order_preconditions(lib, dev):
    """tile_k must be a multiple of 128 dividing the record into whole groups
    of 16 rows, on a 16-byte aligned pair; rejected before any launch."""
    import hipfetch
    h = torch.zeros(4 * 16 * 256, dtype=torch.uint8, pin_memory=True)
    c = torch.zeros(4 * 16 * 256 + 16, dtype=torch.uint8, device=dev)
    src = lib.device_ptr_of(h.data_ptr())
    j = torch.zeros(1, dtype=torch.int32, device=dev)
    for tk, b, d in ((192, 16 * 256, 0), (256, 8 * 256, 0), (256, 16 * 256, 4), (-128, 4096, 0)):
        with pytest.raises(hipfetch.NativeError, match="tile"):
            lib.fetch([(src, c.data_ptr() + d, b, tk)], j, j, j, max_jobs=1, blocks_per_job=1)


@pytest.mark.parametrize("noncoherent", [False, True])
def test_fetch_from_library_host_pool(lib, dev, noncoherent):
    n = 8
    ptr = lib.host_alloc(n * RB, noncoherent=noncoherent)
    try:
        import ctypes
        arr = np.ctypeslib.as_array((ctypes.c_int64 * (n * W64)).from_address(ptr)).reshape(n, W64)
        arr[:] = (np.arange(n, dtype=np.int64)[:, None] << 32) | np.arange(W64, dtype=np.int64)
        cache = torch.full((4 * RB,), 255, dtype=torch.uint8, device=dev)
        fexp = torch.tensor([6, 1, 3, 7], dtype=torch.int32, device=dev)
        fslot = torch.arange(4, dtype=torch.int32, device=dev)
        nmiss = torch.tensor([4], dtype=torch.int32, device=dev)
        say(f"fetch: library host pool noncoherent={noncoherent}")
        lib.fetch([(lib.device_ptr_of(ptr), cache.data_ptr(), RB)], fexp, fslot, nmiss,
                  max_jobs=4, blocks_per_job=32)
        torch.cuda.synchronize()
        assert _check(cache, [6, 1, 3, 7]) == 0
    finally:
        torch.cuda.synchronize()
        lib.host_free(ptr)


def test_is_page_locked_asks_the_runtime(lib, dev):
    """hipfetch.is_page_locked: page-locked torch tensors and the library's
    own host regions (views at an offset too) are page-locked; pageable
    memory, device tensors and empty tensors are not."""
    import ctypes
    assert lib.is_page_locked(torch.empty(1 << 20, dtype=torch.uint8, pin_memory=True))
    assert not lib.is_page_locked(torch.empty(1 << 20, dtype=torch.uint8))
    assert not lib.is_page_locked(torch.empty(1 << 20, dtype=torch.uint8, device=dev))
    assert not lib.is_page_locked(torch.empty(0, dtype=torch.uint8, pin_memory=True))
    n = 64 << 20
    ptr = lib.host_alloc(n)
    try:
        flat = torch.from_numpy(np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(ptr)))
        assert lib.is_page_locked(flat) and lib.is_page_locked(flat[n // 2 + 16:])
    finally:
        lib.host_free(ptr)


def test_pageable_source_is_rejected(lib):
    import hipfetch
    t = torch.empty(1 << 20, dtype=torch.uint8)
    with pytest.raises(hipfetch.NativeError, match="page-locked"):
        lib.device_ptr_of(t.data_ptr())


def test_capture_replays_dynamic_and_honours_job_count(lib, dev, pool):
    """Sets A (warm-up), C (set before capture), B (set before replay): the
    replay must serve B (DYNAMIC); a second replay with nmiss halved must
    leave the surplus slots untouched."""
    jobs = 8
    rng = np.random.default_rng(5)
    perm = rng.permutation(256)
    A, Cs, B = perm[:8].tolist(), perm[8:16].tolist(), perm[16:24].tolist()
    cache = torch.full((jobs * RB,), 255, dtype=torch.uint8, device=dev)
    fexp = torch.tensor(A, dtype=torch.int32, device=dev)
    fslot = torch.arange(jobs, dtype=torch.int32, device=dev)
    nmiss = torch.tensor([jobs], dtype=torch.int32, device=dev)
    src = lib.device_ptr_of(pool.data_ptr())
    pairs = [(src, cache.data_ptr(), RB)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            lib.fetch(pairs, fexp, fslot, nmiss, jobs, 64)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    fexp.copy_(torch.tensor(Cs, dtype=torch.int32))
    g = torch.cuda.CUDAGraph()
    say("fetch: capture")
    with torch.cuda.graph(g):
        lib.fetch(pairs, fexp, fslot, nmiss, jobs, 64)
    cache.fill_(255)
    fexp.copy_(torch.tensor(B, dtype=torch.int32))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert _check(cache, B) == 0, "replay did not serve the replay-time experts"
    cache.fill_(255)
    nmiss.fill_(jobs // 2)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert _check(cache, B[:jobs // 2]) == 0
    assert _untouched(cache, jobs // 2, jobs)


def test_copy_engine_capture_is_frozen_fetch_kernel_dynamic(lib, dev, pool):
    """The premise of the fetch kernel, measured on ROCm with the
    reference's A/C/B protocol (bin/bench_hostread.py:852-934,
    notes/06-cuda-graphs-plan.md:182): a captured copy_ per miss from the
    page-locked pool (hipMemcpyAsync, a memcpy node) resolves the expert to
    a source address when it is captured, so the replay after the ids were
    set to B serves C's records, the capture-time experts (FROZEN); the
    fetch kernel, which reads the ids on the device, serves B (DYNAMIC)."""
    jobs = 4
    A, C_, B = [10, 20, 30, 40], [50, 60, 70, 80], [90, 100, 110, 120]
    src = lib.device_ptr_of(pool.data_ptr())
    records = pool.view(-1, RB)
    results = {}
    for mech in ("copy_", "fetch kernel"):
        cache = torch.full((jobs * RB,), 255, dtype=torch.uint8, device=dev)
        slots = cache.view(jobs, RB)
        ids_live = torch.zeros(jobs, dtype=torch.int32, device=dev)
        ids_host = [0] * jobs
        fslot = torch.arange(jobs, dtype=torch.int32, device=dev)
        nmiss = torch.tensor([jobs], dtype=torch.int32, device=dev)

        def set_ids(ids):
            ids_host[:] = ids
            ids_live.copy_(torch.tensor(ids, dtype=torch.int32))

        def run():
            if mech == "copy_":
                for j, e in enumerate(ids_host):
                    slots[j].copy_(records[e], non_blocking=True)
            else:
                lib.fetch([(src, cache.data_ptr(), RB)], ids_live, fslot, nmiss, max_jobs=jobs,
                          blocks_per_job=2)

        say(f"A/C/B capture protocol: {mech}")
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                set_ids(A)
                run()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        set_ids(C_)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            run()
        cache.fill_(255)
        set_ids(B)
        g.replay()
        torch.cuda.synchronize()
        if _check(cache, B) == 0:
            results[mech] = "DYNAMIC"
        elif _check(cache, C_) == 0:
            results[mech] = "FROZEN"
        elif bool((cache == 255).all()):
            results[mech] = "untouched (the replay did nothing)"
        else:
            results[mech] = "WRONG"
        del g
    print(f"A/C/B on MI355X: {results}")
    assert results == {"copy_": "FROZEN", "fetch kernel": "DYNAMIC"}
