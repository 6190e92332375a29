"""Fetch of entropy-coded records on the GPU: the cache slots it fills equal
the raw records byte for byte (the closed form: decoding is the identity on
the stored bytes), for miss lists read on the device, under graph replay
with the lists changing, and for a record layout with a padded tail."""
import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu


def _raw_records(n, H, I, seed):
    import synth
    from hostpool import RecordLayout
    lay = RecordLayout(H, I)
    g = torch.Generator(device="cpu").manual_seed(seed)
    w13, s13 = synth.quantize_blocks(torch.randn((n, 2 * I, H), generator=g) * 0.02)
    w2, s2 = synth.quantize_blocks(torch.randn((n, H, I), generator=g) * 0.02)
    rec = lay.pack(w13, s13, w2, s2).numpy()
    if lay.record_bytes > lay.payload_bytes:
        rec[:, lay.payload_bytes:] = np.arange(lay.record_bytes - lay.payload_bytes) % 251
    return lay, rec


@pytest.mark.parametrize("H,I,n,workgroups", [(2048, 512, 24, 32), (256, 128, 40, 3)])
def test_coded_fetch_fills_slots_with_the_raw_records(lib, dev, H, I, n, workgroups):
    import codec
    lay, raw = _raw_records(n, H, I, H + n)
    pool = codec.CodedPool(raw, lay, dev)
    say(f"coded fetch: H={H} I={I} n={n} ratio {pool.ratio:.4f}")
    C = 12
    cache = torch.zeros((C, lay.record_bytes), dtype=torch.uint8, device=dev)
    rng = np.random.default_rng(7)
    try:
        for jobs in (1, 3, 8):
            experts = rng.choice(n, jobs, replace=False)
            slots = rng.choice(C, jobs, replace=False)
            cache.fill_(0xAB)
            # lists of max_jobs entries, the tail past the jobs never read
            fe = torch.full((8,), -1, dtype=torch.int32, device=dev)
            fs = torch.full((8,), -1, dtype=torch.int32, device=dev)
            fe[:jobs] = torch.tensor(experts, dtype=torch.int32)
            fs[:jobs] = torch.tensor(slots, dtype=torch.int32)
            nm = torch.tensor([jobs], dtype=torch.int32, device=dev)
            pool.fetch(cache, fe, fs, nm, max_jobs=8, workgroups=workgroups)
            torch.cuda.synchronize()
            got = cache.cpu().numpy()
            for e, s in zip(experts, slots):
                assert np.array_equal(got[s], raw[e]), f"slot {s} != record {e} (jobs {jobs})"
            for s in set(range(C)) - set(slots.tolist()):
                assert (got[s] == 0xAB).all(), f"slot {s} written without a job"
    finally:
        pool.close()


def test_coded_fetch_in_a_graph_with_changing_lists(lib, dev):
    import codec
    lay, raw = _raw_records(16, 2048, 512, 11)
    pool = codec.CodedPool(raw, lay, dev)
    C = 8
    cache = torch.zeros((C, lay.record_bytes), dtype=torch.uint8, device=dev)
    fe = torch.zeros(8, dtype=torch.int32, device=dev)
    fs = torch.zeros(8, dtype=torch.int32, device=dev)
    nm = torch.zeros(1, dtype=torch.int32, device=dev)
    try:
        s = torch.cuda.Stream(device=dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s):
            pool.fetch(cache, fe, fs, nm, max_jobs=8)
        torch.cuda.current_stream(dev).wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            pool.fetch(cache, fe, fs, nm, max_jobs=8)
        rng = np.random.default_rng(3)
        for r in range(5):
            jobs = int(rng.integers(0, 9))
            experts = rng.choice(16, jobs, replace=False)
            slots = rng.choice(C, jobs, replace=False)
            fe[:jobs] = torch.tensor(experts, dtype=torch.int32)
            fs[:jobs] = torch.tensor(slots, dtype=torch.int32)
            nm.fill_(jobs)
            cache.zero_()
            torch.cuda.synchronize()
            say(f"coded fetch graph replay {r}: {jobs} jobs")
            g.replay()
            torch.cuda.synchronize()
            got = cache.cpu().numpy()
            for e, sl in zip(experts, slots):
                assert np.array_equal(got[sl], raw[e]), (r, e, sl)
            for sl in set(range(C)) - set(slots.tolist()):
                assert not got[sl].any()
    finally:
        pool.close()


@pytest.mark.parametrize("mode", ["cached", "nocache"])
def test_decode_step_with_coded_pools_equals_raw_pools(lib, dev, mode):
    """The captured decode step fetching from coded pools fills the same cache
    slots with the same bytes, so every step's output and the caches equal
    the raw-pool step's."""
    import decode
    cfg = decode.DecodeConfig(layers=3, n_experts=32, top_k=4, hidden=512, inter=256,
                              capacity=10, schedule_steps=8, drift_every=4, gate_std=0.02,
                              mode=mode)
    raw = decode.DecodeHarness(cfg, dev)
    cfgc = decode.DecodeConfig(**{**cfg.__dict__, "coded_pool": True, "coded_workgroups": 5})
    cod = decode.DecodeHarness(cfgc, dev, pools=raw.pools)
    try:
        say(f"coded decode ({mode}): ratio {np.mean([c.ratio for c in cod.coded]):.4f}")
        raw.capture()
        cod.capture()
        for s in range(6):
            raw.replay(1)
            cod.replay(1)
            torch.cuda.synchronize()
            assert torch.equal(cod.x, raw.x), f"step {s}"
        for l in range(cfg.layers):
            assert torch.equal(cod.cache[l], raw.cache[l]), f"layer {l} cache"
        assert cod.hit_rate() == raw.hit_rate()
    finally:
        cod.pools = []
        cod.close()
        raw.close()
