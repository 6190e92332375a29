"""The single-layer, single-token decode workload end to end on the GPU:
256 experts (N(0, 0.02) weights, 128x128 block-quantised) in a page-locked
pool of packed records, an empty 64-slot device cache, x ~ N(0, 1), router
W ~ N(0, 0.02), seed 0.  Every routed expert misses, so one step fetches
8 x 3,146,496 = 25,171,968 bytes.  Checked against the oracle: router ids
bit for bit, slot choices and miss queue, the fetched records byte for byte,
and the MoE output within 1e-2 of the W8A8 restatement (the W8A16 gap is
reported); with the activations kept in bf16 (fp8_moe_forward mode 3) the
output is within 1e-2 of the dequantise-then-matmul closed form."""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import moe as omoe
from oracle import router as orouter
from oracle import slots as oslots

pytestmark = pytest.mark.gpu
E, H, I, K, C = 256, 2048, 512, 8, 64


def test_single_layer_decode_all_miss(lib, dev):
    import decode
    import synth
    from hostpool import DRAMA3, HostPool
    lay = DRAMA3
    RB = lay.record_bytes
    say("config 0: filling the 256-record pinned pool")
    pool = HostPool(E, lay)
    try:
        decode.fill_pool_on_gpu(pool, seed=0, layer=0, device=dev)
        gate = synth.router_weight(0).to(dev)
        x = synth.hidden_states(0, 1).to(dev)
        i32 = dict(dtype=torch.int32, device=dev)
        slot_of, slot_expert = torch.empty(E, **i32), torch.empty(C, **i32)
        stamp = torch.empty(C, dtype=torch.int64, device=dev)
        step = torch.empty(1, dtype=torch.int64, device=dev)
        lib.slots_init(slot_of, slot_expert, stamp, step)
        cache = torch.zeros((C, RB), dtype=torch.uint8, device=dev)
        ids, wts = torch.zeros((1, K), **i32), torch.zeros((1, K), dtype=torch.float32, device=dev)
        logits = torch.zeros((1, E), dtype=torch.float32, device=dev)
        out_slot, fslot, fexp = (torch.zeros(K, **i32) for _ in range(3))
        nmiss = torch.zeros(1, **i32)
        say("config 0: route + resolve, fetch, expert FFN")
        lib.route_resolve(x, gate, None, K, logits, ids, wts, slot_of, slot_expert, stamp, step,
                          out_slot, fslot, fexp, nmiss, None)
        lib.fetch([(pool.dev_ptr, cache.data_ptr(), RB)], fexp, fslot, nmiss, max_jobs=K,
                  blocks_per_job=2)
        out = torch.empty_like(x)
        ws = torch.empty(lib.fp8_moe_workspace(1, K, C, H, I), dtype=torch.uint8, device=dev)
        lib.fp8_moe_forward(x, out_slot.view(1, K), wts, *lay.views(cache), out, ws,
                            layout=lay.code)
        out16 = torch.empty_like(x)          # mode 3: bf16 activations
        lib.fp8_moe_forward(x, out_slot.view(1, K), wts, *lay.views(cache), out16, ws, mode=3,
                            layout=lay.code)
        torch.cuda.synchronize()

        o_ids, o_w, _ = orouter.route(x.float().cpu().numpy(), gate.float().cpu().numpy(), K)
        assert np.array_equal(ids.cpu().numpy(), o_ids)
        assert np.allclose(wts.cpu().numpy(), o_w, rtol=1e-6, atol=1e-7)
        tab = oslots.SlotTable.fresh(E, C)
        o_slots, o_fs, o_fe = oslots.resolve(tab, o_ids[0].tolist())
        assert out_slot.tolist() == o_slots
        assert int(nmiss) == K and fslot.tolist() == o_fs and fexp.tolist() == o_fe
        recs = pool.tensor
        fetched = 0
        for s, e in zip(o_slots, o_ids[0].tolist()):
            assert torch.equal(cache[s].cpu(), recs[e]), f"slot {s} != record {e}"
            fetched += RB
        assert fetched == 25_171_968

        # the oracle gets the 8 routed records only, ids renumbered 0..7
        sel = recs[torch.from_numpy(o_ids[0].astype(np.int64))].clone()
        d13, ds13, d2, ds2 = lay.unpack(sel.numpy())
        args = (x.float().cpu().numpy(), np.arange(K)[None, :],
                wts.cpu().numpy().astype(np.float64), d13, ds13, d2, ds2)
        got = out.float().cpu().numpy()
        err = omoe.max_rel_err(got, omoe.forward_w8a8(*args))
        gap = omoe.max_rel_err(got, omoe.forward_w8a16(*args))
        gap16 = omoe.max_rel_err(out16.float().cpu().numpy(), omoe.forward_w8a16(*args))
        print(f"config 0: ids {ids[0].tolist()}, max rel err vs W8A8 {err:.2e}, "
              f"vs dequantise path {gap:.2e}; bf16-activation mode vs dequantise path "
              f"{gap16:.2e}")
        assert err <= 1e-2
        assert gap <= 6e-2          # the activation quantisation error, 4.5e-2 measured
        assert gap16 <= 1e-2        # mode 3 keeps the activations in bf16
    finally:
        pool.close()
