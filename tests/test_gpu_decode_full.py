"""The 40-layer decode step at its real shape, checked layer by layer.

Workload: 40 layers, 256 experts of H 2048 / I 512 in fp8 e4m3 with
128 x 128 block scales, top-8 routing (bf16 gate logits plus the per-layer
Zipf popularity bias), a 50-slot device cache per layer (~60 % hit), the
expert records in 40 page-locked host pools, and the whole step captured in
one hipGraph.  Popularity is redrawn every 4 steps, so the 6 steps run here
cross a drift boundary.

Eager steps, for every layer of every step:
  * router ids bit-exact against oracle.router (weights within float32
    rounding), on the layer's own hidden state;
  * out_slot, fetch_slot and fetch_expert equal to oracle.slots.resolve on a
    per-layer oracle table, and the device hit/miss counters equal to the
    oracle's;
  * every record fetched into the cache byte-equal to its host record;
  * the layer output equal, bit for bit, to h + the expert FFN's output
    (the residual add fused into the down kernel), and on 4 sampled layers
    per step that FFN output within 1e-2 (max rel err) of the W8A8 oracle.
At the end of the eager steps every occupied slot of every layer holds its
expert's record, and the tables equal the oracle's.

Graph: the captured step, replayed over the same 6 schedule steps from empty
caches, gives bit for bit the eager steps' outputs, tables and counters.

Reference behaviour followed: bin/test_devcache.py:47-133 (cache path
against the kernel on the same inputs, exact, DYNAMIC replay),
bin/devcache.py:230-277 (the decode step).
"""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import moe as omoe
from oracle import router as orouter
from oracle import slots as oslots

pytestmark = pytest.mark.gpu

L, E, K, H, I, C = 40, 256, 8, 2048, 512, 50
STEPS = 6
TOL = 1e-2


def _unpack(layout, recs: np.ndarray):
    """Packed records [n, record] -> dense (w13 codes [n,2I,H], s13, w2 codes [n,H,I], s2)."""
    return layout.unpack(recs)


def _tables(hx, l):
    return (hx.slot_of[l].cpu().numpy(), hx.slot_expert[l].cpu().numpy(),
            hx.stamp[l].cpu().numpy(), int(hx.step[l].item()))


@pytest.mark.timeout(900)
def test_full_shape_decode_step_eager_and_graph(lib, dev):
    from decode import DecodeConfig, DecodeHarness
    cfg = DecodeConfig(layers=L, n_experts=E, top_k=K, hidden=H, inter=I, capacity=C,
                       drift_every=4, schedule_steps=8)
    say("decode-full: building 40 page-locked pools of 256 records (30 GiB)")
    hx = DecodeHarness(cfg, dev)
    try:
        lay = hx.layout
        # device copy of every pool, to compare cache slots against on the GPU
        pool_dev = [torch.from_numpy(p.array).to(dev) for p in hx.pools]
        gate_np = [hx.gate[l].float().cpu().numpy() for l in range(L)]
        ws = torch.empty(lib.fp8_moe_workspace(1, K, C, H, I), dtype=torch.uint8, device=dev)
        y = torch.empty((1, H), dtype=torch.bfloat16, device=dev)
        otab = [oslots.SlotTable.fresh(E, C) for _ in range(L)]
        ohits = np.zeros((L, 2), np.int64)
        rng = np.random.default_rng(5)
        eager = []
        hx.restart()
        for s in range(STEPS):
            sampled = set(rng.choice(L, 4, replace=False).tolist())
            say(f"decode-full: eager step {s}, FFN checked on layers {sorted(sampled)}")
            hx.stage(s)
            bias_np = hx.bias_live.cpu().numpy()
            hx.x.copy_(hx.x0)
            for l in range(L):
                hx.layer(l)
                torch.cuda.synchronize(dev)
                h = hx.h.clone()
                # router: ids bit-exact, weights within float32 rounding
                o_ids, o_w, _ = orouter.route(h.float().cpu().numpy(), gate_np[l], K,
                                              bias_np[l], "bf16")
                ids = hx.ids[l].cpu().numpy()
                assert np.array_equal(ids, o_ids), f"step {s} layer {l}: router ids"
                np.testing.assert_allclose(hx.wts[l].cpu().numpy(), o_w, rtol=2e-6, atol=1e-7)
                # slot decisions and miss queue
                want_out, want_fs, want_fe = oslots.resolve(otab[l], o_ids[0].tolist())
                n = int(hx.nmiss[l].item())
                assert hx.out_slot[l].view(-1).tolist() == want_out, f"step {s} layer {l}"
                assert hx.fslot[l][:n].tolist() == want_fs, f"step {s} layer {l}"
                assert hx.fexp[l][:n].tolist() == want_fe, f"step {s} layer {l}"
                ohits[l] += (K - n, n)
                # fetched records byte-exact
                for j in range(n):
                    sl, e = want_fs[j], want_fe[j]
                    assert torch.equal(hx.cache[l][sl], pool_dev[l][e]), \
                        f"step {s} layer {l}: slot {sl} does not hold expert {e}"
                # the layer's output is h + FFN(h), the add exact in bf16
                w13, s13, w2, s2 = hx.views[l]
                lib.fp8_moe_forward(h, hx.out_slot[l], hx.wts[l], w13, s13, w2, s2, y, ws,
                                    layout=lay.code)
                torch.cuda.synchronize(dev)
                assert torch.equal((h + y).view(torch.int16), hx.x.view(torch.int16)), \
                    f"step {s} layer {l}: fused residual"
                if l in sampled:
                    dense = _unpack(lay, hx.pools[l].array[np.asarray(o_ids[0])])
                    want = omoe.forward_w8a8(h.float().cpu().numpy(), np.arange(K)[None, :],
                                             hx.wts[l].cpu().numpy().astype(np.float64), *dense)
                    err = omoe.max_rel_err(y.float().cpu().numpy(), want)
                    say(f"decode-full: step {s} layer {l}: FFN max rel err {err:.2e}")
                    assert err <= TOL
            eager.append(dict(x=hx.x.clone(), stats=hx.stats.clone(),
                              tables=[_tables(hx, l) for l in range(L)]))
        # counters and tables against the oracle after the last step
        assert np.array_equal(hx.stats.cpu().numpy(), ohits)
        for l in range(L):
            so, se, st, stp = _tables(hx, l)
            o_so, o_se, o_st, o_stp = otab[l].arrays()
            assert np.array_equal(so, o_so) and np.array_equal(se, o_se)
            assert np.array_equal(st, o_st) and stp == int(o_stp)
            for sl in np.nonzero(se >= 0)[0].tolist():
                assert torch.equal(hx.cache[l][sl], pool_dev[l][int(se[sl])]), \
                    f"layer {l}: slot {sl}"
        hit = ohits[:, 0].sum() / ohits.sum()
        say(f"decode-full: eager steps match the oracle; hit rate {hit:.3f}")

        # the captured step replays the same schedule from empty caches
        say("decode-full: capturing the 40-layer step")
        hx.capture()
        for s in range(STEPS):
            say(f"decode-full: graph replay {s}")
            hx.replay(1)
            torch.cuda.synchronize(dev)
            want = eager[s]
            assert torch.equal(hx.x.view(torch.int16), want["x"].view(torch.int16)), \
                f"replay {s}: output differs from the eager step"
            assert torch.equal(hx.stats, want["stats"]), f"replay {s}: counters"
            for l in range(L):
                got = _tables(hx, l)
                exp = want["tables"][l]
                assert all(np.array_equal(a, b) for a, b in zip(got[:3], exp[:3])) and \
                    got[3] == exp[3], f"replay {s} layer {l}: table"
        assert torch.isfinite(hx.x.float()).all()
    finally:
        hx.close()
