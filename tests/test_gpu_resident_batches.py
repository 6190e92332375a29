"""All-resident batched decode at the workload's batch sizes: 256 experts of
H 2048 / I 512 in HBM (packed records), B = 8, 32 and 128 tokens per step,
top-8 routing through the router kernel (bf16 gate logits), then the expert
FFN on the kernel the automatic choice takes (per-pair GEMV up to 16 tokens,
grouped beyond), with the residual fused.

Checked: router ids bit-exact against oracle.router for every token; the FFN
output of 6 sampled tokens per batch within 2e-2 (max rel err) of the W8A8
oracle on those tokens' 8 experts; the residual add exact in bf16 on every
token; both kernel paths forced on the same inputs give bit-identical rows.
"""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import moe as omoe
from oracle import router as orouter

pytestmark = pytest.mark.gpu
E, H, I, K = 256, 2048, 512, 8
TOL = 2e-2


@pytest.fixture(scope="module")
def resident(dev):
    import synth
    from hostpool import DRAMA3
    g = torch.Generator(device=dev).manual_seed(21)
    rec = torch.empty((E, DRAMA3.record_bytes), dtype=torch.uint8, device=dev)
    for e0 in range(0, E, 64):
        w13, s13 = synth.quantize_blocks(torch.randn((64, 2 * I, H), generator=g, device=dev) * 0.02)
        w2, s2 = synth.quantize_blocks(torch.randn((64, H, I), generator=g, device=dev) * 0.02)
        rec[e0:e0 + 64] = DRAMA3.pack(w13, s13, w2, s2)
    gate = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    return rec, gate


def _unpack(rec_np):
    from hostpool import DRAMA3
    return DRAMA3.unpack(rec_np)


@pytest.mark.parametrize("B", [8, 32, 128])
def test_resident_batch_against_oracle(lib, dev, resident, B):
    import moe
    import synth
    from hostpool import DRAMA3
    rec, gate = resident
    views = DRAMA3.views(rec)
    x = synth.hidden_states(100 + B, B).to(dev)
    say(f"resident: B={B} route")
    ids, wts, _ = moe.route(x, gate, K, ids_dtype=torch.int32)
    torch.cuda.synchronize()
    o_ids, o_w, _ = orouter.route(x.float().cpu().numpy(), gate.float().cpu().numpy(), K)
    assert np.array_equal(ids.cpu().numpy(), o_ids)
    np.testing.assert_allclose(wts.cpu().numpy(), o_w, rtol=2e-6, atol=1e-7)
    say(f"resident: B={B} expert FFN ({'GEMV' if B <= 16 else 'grouped'})")
    ws = torch.empty(lib.fp8_moe_workspace(B, K, E, H, I), dtype=torch.uint8, device=dev)
    outs = {}
    for mode in (0, 1, 2):
        y = torch.empty_like(x)
        lib.fp8_moe_forward(x, ids, wts, *views, y, ws, mode=mode, layout=DRAMA3.code)
        outs[mode] = y
    res = torch.empty_like(x)
    lib.fp8_moe_forward(x, ids, wts, *views, res, ws, residual=x, layout=DRAMA3.code)
    torch.cuda.synchronize()
    assert torch.equal(outs[1].view(torch.int16), outs[2].view(torch.int16)), "GEMV != grouped"
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert torch.equal((x + outs[0]).view(torch.int16), res.view(torch.int16)), "residual"
    assert torch.isfinite(outs[0].float()).all()
    rng = np.random.default_rng(B)
    for t in sorted(rng.choice(B, 6, replace=False).tolist()):
        sel = o_ids[t]
        dense = _unpack(rec[torch.from_numpy(sel.astype(np.int64)).to(dev)].cpu().numpy())
        want = omoe.forward_w8a8(x[t:t + 1].float().cpu().numpy(), np.arange(K)[None, :],
                                 wts[t:t + 1].cpu().numpy().astype(np.float64), *dense)
        err = omoe.max_rel_err(outs[0][t:t + 1].float().cpu().numpy(), want)
        say(f"resident: B={B} token {t}: max rel err {err:.2e}")
        assert err <= TOL


def test_resident_batch1_fused_launch_against_oracle(lib, dev, resident):
    """Batch 1 on the decode step's fused launch (moe_route_fetch_ffn over
    the 256 resident records with a table that holds every expert: route +
    gate/up in one launch, then down): no miss is ever queued; router ids
    bit-exact against oracle.router; the output equals the separate router
    + GEMV launches bit for bit (with and without the residual) and the
    W8A8 oracle within 1e-2, token after token."""
    import decode
    import moe
    import synth
    from hostpool import DRAMA3
    rec, gate = resident
    views = DRAMA3.views(rec)
    so, se, st, step = decode.resident_table(E, dev)
    i32 = dict(dtype=torch.int32, device=dev)
    logits = torch.empty((1, E), dtype=torch.float32, device=dev)
    ids = torch.empty((1, K), **i32)
    wts = torch.empty((1, K), dtype=torch.float32, device=dev)
    out_slot, fslot, fexp = (torch.empty(K, **i32) for _ in range(3))
    nmiss = torch.empty(1, **i32)
    stats = torch.zeros(2, dtype=torch.int64, device=dev)
    ws = torch.empty(lib.fp8_moe_workspace(1, K, E, H, I), dtype=torch.uint8, device=dev)
    for t in range(4):
        x = synth.hidden_states(300 + t, 1).to(dev)
        outs = {}
        for res in (None, x):
            o = torch.empty_like(x)
            lib.route_fetch_ffn(x, gate, None, K, logits, ids, wts, so, se, st, step, out_slot,
                                fslot, fexp, nmiss, rec.data_ptr(), rec, I, 4, o, ws,
                                residual=res, stats=stats)
            outs[res is None] = o
        say(f"resident B=1 fused: token {t}")
        r_ids, r_w, _ = moe.route(x, gate, K, ids_dtype=torch.int32)
        sep = torch.empty_like(x)
        sep_res = torch.empty_like(x)
        lib.fp8_moe_forward(x, r_ids, r_w, *views, sep, ws, mode=1, layout=DRAMA3.code)
        lib.fp8_moe_forward(x, r_ids, r_w, *views, sep_res, ws, mode=1, residual=x,
                            layout=DRAMA3.code)
        torch.cuda.synchronize()
        assert int(nmiss[0]) == 0
        assert torch.equal(ids, r_ids) and torch.equal(out_slot.view(1, K), ids)
        o_ids, o_w, _ = orouter.route(x.float().cpu().numpy(), gate.float().cpu().numpy(), K)
        assert np.array_equal(ids.cpu().numpy(), o_ids)
        assert torch.equal(outs[True].view(torch.int16), sep.view(torch.int16))
        assert torch.equal(outs[False].view(torch.int16), sep_res.view(torch.int16))
        dense = _unpack(rec[torch.from_numpy(o_ids[0].astype(np.int64)).to(dev)].cpu().numpy())
        want = omoe.forward_w8a8(x.float().cpu().numpy(), np.arange(K)[None, :],
                                 wts.cpu().numpy().astype(np.float64), *dense)
        err = omoe.max_rel_err(outs[True].float().cpu().numpy(), want)
        assert err <= 1e-2, f"token {t}: max rel err {err:.2e}"
    assert stats.tolist() == [8 * 8, 0]


@pytest.mark.parametrize("shape", [
    dict(E=256, K=8, H=2048, I=512, T=1, bias=False),
    dict(E=256, K=8, H=2048, I=512, T=8, bias=False),
    # the GEMV path's most tokens
    dict(E=256, K=8, H=2048, I=512, T=16, bias=True),
    # the 16-per-lane logits (E > 256), the largest top_k, a router bias
    dict(E=320, K=16, H=1024, I=256, T=1, bias=True),
    dict(E=320, K=16, H=1024, I=256, T=5, bias=True),
    dict(E=1024, K=4, H=512, I=128, T=3, bias=True),
], ids=["drama3", "drama3_t8", "drama3_t16", "e320_top16", "e320_top16_t5", "e1024_t3"])
def test_resident_router_in_gateup_equals_separate_launches(lib, dev, resident, shape):
    """moe_router_fp8_moe_forward (the logits launch, then the top-k made by
    every wave of the gate/up launch, then down) against moe_router_topk +
    moe_fp8_moe_forward(mode 1), for 1 to 16 tokens: logits, ids, weights
    and the output (with and without the residual) bit for bit, batch after
    batch, eager and replayed from a graph; at Drama-3 shape the ids against
    oracle.router and the first tokens' output against the W8A8 oracle
    within 1e-2."""
    import moe
    import synth
    from hostpool import DRAMA3, RecordLayout
    E_, K_, H_, I_, T_ = shape["E"], shape["K"], shape["H"], shape["I"], shape["T"]
    if E_ == E:
        rec, gate = resident
        lay = DRAMA3
    else:
        lay = RecordLayout(H_, I_)
        g = torch.Generator(device=dev).manual_seed(E_ + K_)
        w13, s13 = synth.quantize_blocks(torch.randn((E_, 2 * I_, H_), generator=g, device=dev) * 0.02)
        w2, s2 = synth.quantize_blocks(torch.randn((E_, H_, I_), generator=g, device=dev) * 0.02)
        rec = lay.pack(w13, s13, w2, s2)
        gate = (torch.randn((E_, H_), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    views = lay.views(rec)
    bias = (torch.randn(E_, generator=torch.Generator().manual_seed(5)) * 0.01).to(dev) \
        if shape["bias"] else None
    i32 = dict(dtype=torch.int32, device=dev)
    ws = torch.empty(lib.fp8_moe_workspace(T_, K_, E_, H_, I_), dtype=torch.uint8, device=dev)
    xs = [synth.hidden_states(500 + t, T_, H_).to(dev) for t in range(4)]
    x = torch.empty_like(xs[0])
    logits = torch.empty((T_, E_), dtype=torch.float32, device=dev)
    ids = torch.empty((T_, K_), **i32)
    wts = torch.empty((T_, K_), dtype=torch.float32, device=dev)
    outs = [torch.empty_like(x) for _ in range(2)]

    def fused():
        for o, res in zip(outs, (None, x)):
            lib.router_fp8_moe_forward(x, gate, bias, K_, logits, ids, wts, *views, o, ws,
                                       residual=res, layout=lay.code)

    def separate():
        r_logits = torch.empty((T_, E_), dtype=torch.float32, device=dev)
        r_ids = torch.empty((T_, K_), **i32)
        r_w = torch.empty((T_, K_), dtype=torch.float32, device=dev)
        lib.router_topk(x, gate, bias, K_, r_logits, r_ids, r_w)
        sep = [torch.empty_like(x) for _ in range(2)]
        for o, res in zip(sep, (None, x)):
            lib.fp8_moe_forward(x, r_ids, r_w, *views, o, ws, mode=1, residual=res,
                                layout=lay.code)
        return r_logits, r_ids, r_w, sep

    def check(tag):
        r_logits, r_ids, r_w, sep = separate()
        torch.cuda.synchronize()
        assert torch.equal(logits, r_logits), f"{tag}: logits"
        assert torch.equal(ids, r_ids), f"{tag}: ids"
        assert torch.equal(wts, r_w), f"{tag}: weights"
        for o, s_, name in zip(outs, sep, ("out", "out + residual")):
            assert torch.equal(o.view(torch.int16), s_.view(torch.int16)), f"{tag}: {name}"
        if E_ == E and bias is None:
            o_ids, _, _ = orouter.route(x.float().cpu().numpy(), gate.float().cpu().numpy(), K_)
            assert np.array_equal(ids.cpu().numpy(), o_ids), tag
            for t in range(min(T_, 2)):
                dense = _unpack(rec[ids[t].long()].cpu().numpy())
                want = omoe.forward_w8a8(x[t:t + 1].float().cpu().numpy(),
                                         np.arange(K_)[None, :],
                                         wts[t:t + 1].cpu().numpy().astype(np.float64), *dense)
                err = omoe.max_rel_err(outs[0][t:t + 1].float().cpu().numpy(), want)
                assert err <= 1e-2, f"{tag} token {t}: max rel err {err:.2e}"

    for t, xt in enumerate(xs):
        x.copy_(xt)
        say(f"router in gate/up {shape}: eager token {t}")
        fused()
        check(f"eager {t}")
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        fused()
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fused()
    for t, xt in enumerate(reversed(xs)):
        x.copy_(xt)
        for o in outs:
            o.fill_(float("nan"))
        say(f"router in gate/up {shape}: replay {t}")
        graph.replay()
        check(f"replay {t}")
    del graph
