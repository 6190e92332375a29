"""Loader into page-locked pools on the GPU box: pools built from safetensors
shards hold the packed records byte for byte, and the expert FFN over records
fetched from those pools equals the FFN over the reference-layout buffers
loaded from the same shards, bit for bit."""
import numpy as np
import pytest
import torch

from conftest import say
from test_loader import _write_shards

pytestmark = pytest.mark.gpu


def test_pools_from_shards_feed_the_fetch_and_ffn(lib, dev, tmp_path):
    import loader
    import moe
    from hostpool import RecordLayout
    E, H, I, K = 6, 256, 128, 4
    _write_shards(tmp_path, layers=2, E=E, H=H, I=I, seed=9)
    lay = RecordLayout(H, I)
    say("loader: pools from shards")
    pools, nbytes = loader.load_host_pools(tmp_path, [0, 1], lay, threads=4)
    try:
        assert nbytes == 2 * E * lay.payload_bytes
        index = loader.ShardIndex.from_dir(tmp_path)
        ref = moe.MoEExperts(E, H, I)
        loader.fill_expert_buffers(index, 1, ref)
        want_rec = lay.pack(ref.w13_weight, ref.w13_scale_inv, ref.w2_weight, ref.w2_scale_inv)
        assert np.array_equal(pools[1].array, want_rec.numpy())
        cache = torch.zeros((E, lay.record_bytes), dtype=torch.uint8, device=dev)
        order = torch.tensor([3, 0, 5, 1, 4, 2], dtype=torch.int32, device=dev)
        slots = torch.arange(E, dtype=torch.int32, device=dev)
        n = torch.tensor([E], dtype=torch.int32, device=dev)
        lib.fetch([pools[1].fetch_pair(cache)], order, slots, n, max_jobs=E, blocks_per_job=2)
        x = torch.randn((5, H), device=dev).to(torch.bfloat16)
        ids = torch.tensor([[0, 1, 2, 3], [5, 4, 3, 2], [1, 3, 5, 0], [2, 2, 2, 2], [4, 0, 1, 5]],
                           device=dev)
        w = torch.full((5, K), 0.25, device=dev)
        from fp8_moe import fp8_moe_forward
        resident = ref.to(dev)
        want = fp8_moe_forward(x, ids, w, resident.w13_weight, resident.w13_scale_inv,
                               resident.w2_weight, resident.w2_scale_inv)
        # slot s of the cache holds expert order[s]
        slot_of = torch.empty(E, dtype=torch.long, device=dev)
        slot_of[order.long()] = torch.arange(E, device=dev)
        # tile-ordered records against the module's row-major buffers: bit for bit
        got = fp8_moe_forward(x, slot_of[ids], w, *lay.views(cache), layout=lay.code)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
    finally:
        for p in pools:
            p.close()
