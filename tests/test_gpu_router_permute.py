"""Router and permute/unpermute on the GPU: expert ids and orderings
bit-exact against the oracle, weights within float32 rounding."""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import permute as operm
from oracle import router as orouter

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("logit_dtype", ["bf16", "f32"])
@pytest.mark.parametrize("T", [1, 7, 64, 512])
def test_router_ids_bit_exact(lib, dev, T, logit_dtype):
    import moe
    import synth
    x = synth.hidden_states(T, T).to(dev)
    w = synth.router_weight(T).to(dev)
    say(f"router: T={T}, {logit_dtype} logits")
    ids, wts, logits = moe.route(x, w, 8, logit_dtype=logit_dtype)
    torch.cuda.synchronize()
    o_ids, o_w, o_lg = orouter.route(x.float().cpu().numpy(), w.float().cpu().numpy(), 8,
                                     logit_dtype=logit_dtype)
    assert np.array_equal(logits.cpu().numpy(), o_lg)
    assert np.array_equal(ids.cpu().numpy(), o_ids)
    np.testing.assert_allclose(wts.cpu().numpy(), o_w, rtol=2e-6, atol=1e-7)


def test_router_with_bias_int32_bf16_outputs(lib, dev):
    import moe
    import synth
    T = 16
    x = synth.hidden_states(1, T).to(dev)
    w = synth.router_weight(1).to(dev)
    rng = np.random.default_rng(0)
    bias = torch.from_numpy(synth.decode_route_bias(rng, 1, 1)[0, 0]).to(dev)
    ids, wts, logits = moe.route(x, w, 8, bias=bias, ids_dtype=torch.int32,
                                 weights_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    o_ids, o_w, o_lg = orouter.route(x.float().cpu().numpy(), w.float().cpu().numpy(), 8,
                                     bias.cpu().numpy())
    assert np.array_equal(ids.cpu().numpy(), o_ids)
    np.testing.assert_allclose(wts.float().cpu().numpy(), o_w, rtol=8e-3)


def test_router_bf16_tie_goes_to_the_lower_expert(lib, dev):
    """Logits 1 + 2^-10 (expert 3) and 1 + 2^-11 (expert 1) round to the
    same bf16 value: expert 1 ranks first; with float32 logits expert 3."""
    import moe
    H, E = 128, 64
    x = torch.zeros((1, H), dtype=torch.bfloat16, device=dev)
    x[0, 0], x[0, 1], x[0, 2] = 1.0, 2.0 ** -10, 2.0 ** -11
    w = torch.zeros((E, H), dtype=torch.bfloat16, device=dev)
    w[3, 0], w[3, 1] = 1.0, 1.0
    w[1, 0], w[1, 2] = 1.0, 1.0
    w[5, 0] = 0.5
    say("router: bf16 tie")
    ids, _, lg = moe.route(x, w, 2)
    ids32, _, lg32 = moe.route(x, w, 2, logit_dtype="f32")
    torch.cuda.synchronize()
    assert lg[0, 1].item() == lg[0, 3].item() == 1.0 and ids.tolist() == [[1, 3]]
    assert lg32[0, 3].item() == 1.0 + 2.0 ** -10 and ids32.tolist() == [[3, 1]]


def test_router_tie_break_lower_index(lib, dev):
    import moe
    H, E = 128, 64
    x = torch.zeros((1, H), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((E, H), dtype=torch.bfloat16, device=dev)
    bias = torch.zeros(E, device=dev)
    bias[[3, 9, 40, 41, 50]] = 1.0
    bias[[60, 2]] = 0.5
    ids, wts, _ = moe.route(x, w, 8, bias=bias)
    torch.cuda.synchronize()
    assert ids[0].tolist() == [3, 9, 40, 41, 50, 2, 60, 0]


def _ids_cases(traces):
    rows, ids = traces["trace_prefill_rows"], traces["trace_prefill_ids"]
    cases = [ids[:rows[0]].astype(np.int64), ids[rows[0]:rows[0] + rows[1]].astype(np.int64)]
    rng = np.random.default_rng(3)
    cases.append(np.stack([rng.choice(256, 8, replace=False) for _ in range(512)]))
    cases.append(np.array([[17, 3, 200, 5, 6, 7, 8, 9]]))
    cases.append(rng.integers(0, 4096, size=(2000, 8)))
    return cases


def test_permute_and_unique_bit_exact(lib, dev, traces):
    for c, ids_np in enumerate(_ids_cases(traces)):
        E = 4096 if ids_np.max() >= 256 else 256
        T, K = ids_np.shape
        ids = torch.from_numpy(ids_np).to(dev)
        if c % 2:
            ids = ids.int()
        counts = torch.empty(E, dtype=torch.int32, device=dev)
        offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
        sp = torch.empty(T * K, dtype=torch.int32, device=dev)
        pos = torch.empty(T * K, dtype=torch.int32, device=dev)
        nu = torch.empty(1, dtype=torch.int32, device=dev)
        uniq = torch.full((E,), -7, dtype=torch.int32, device=dev)
        rank = torch.empty(E, dtype=torch.int32, device=dev)
        inv = torch.empty(T * K, dtype=torch.int32, device=dev)
        say(f"permute: case {c} T={T} E={E}")
        lib.permute(ids, E, counts, offsets, sp, pos)
        lib.unique_inverse(ids, E, counts, nu, uniq, rank, inv)
        torch.cuda.synchronize()
        oc, oo, osp, opos = operm.permute(ids_np, E)
        assert np.array_equal(counts.cpu().numpy(), oc)
        assert np.array_equal(offsets.cpu().numpy(), oo)
        assert np.array_equal(sp.cpu().numpy(), osp)
        assert np.array_equal(pos.cpu().numpy(), opos)
        u, iv = operm.unique_inverse(ids_np)
        n = int(nu.item())
        assert n == len(u) and np.array_equal(uniq[:n].cpu().numpy(), u)
        assert np.array_equal(inv.cpu().numpy(), iv.reshape(-1))


def test_unpermute_matches_oracle(lib, dev):
    rng = np.random.default_rng(9)
    T, K, H = 33, 8, 2048
    ids_np = np.stack([rng.choice(256, K, replace=False) for _ in range(T)])
    _, _, _, opos = operm.permute(ids_np, 256)
    y = torch.randn((T * K, H), generator=torch.Generator().manual_seed(1))
    w = torch.rand((T, K), generator=torch.Generator().manual_seed(2))
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    lib.unpermute(y.to(dev), torch.from_numpy(opos).to(dev), w.to(dev), out)
    torch.cuda.synchronize()
    want = operm.unpermute(y.numpy(), opos, w.numpy(), K)
    got = out.float().cpu().numpy()
    assert np.abs(got - want).max() <= np.abs(want).max() * 2 ** -8


@pytest.mark.parametrize("logit_dtype", ["bf16", "f32"])
def test_route_resolve_equals_router_then_resolve(lib, dev, logit_dtype):
    """The fused decode entry gives the oracle's router ids/weights and the
    oracle's slot decisions, step after step, tables included."""
    import synth
    from oracle import slots as oslots
    E, H, K, C = 256, 2048, 8, 20
    w = synth.router_weight(7).to(dev)
    rng = np.random.default_rng(3)
    i32 = dict(dtype=torch.int32, device=dev)
    slot_of = torch.empty(E, **i32)
    slot_expert = torch.empty(C, **i32)
    stamp = torch.empty(C, dtype=torch.int64, device=dev)
    step = torch.empty(1, dtype=torch.int64, device=dev)
    stats = torch.zeros(2, dtype=torch.int64, device=dev)
    lib.slots_init(slot_of, slot_expert, stamp, step)
    logits = torch.empty((1, E), device=dev)
    ids = torch.empty((1, K), **i32)
    wts = torch.empty((1, K), device=dev)
    out_slot = torch.empty(K, **i32)
    fs = torch.empty(K, **i32)
    fe = torch.empty(K, **i32)
    nm = torch.empty(1, **i32)
    tab = oslots.SlotTable.fresh(E, C)
    for s in range(30):
        x = synth.hidden_states(500 + s, 1).to(dev)
        bias = torch.from_numpy((rng.gumbel(size=E) * 2).astype(np.float32)).to(dev)
        lib.route_resolve(x, w, bias, K, logits, ids, wts, slot_of, slot_expert, stamp, step,
                          out_slot, fs, fe, nm, stats, logit_dtype=logit_dtype)
        torch.cuda.synchronize()
        o_ids, o_w, o_lg = orouter.route(x.float().cpu().numpy(), w.float().cpu().numpy(), K,
                                         bias.cpu().numpy(), logit_dtype=logit_dtype)
        assert np.array_equal(ids.cpu().numpy(), o_ids), f"step {s}"
        np.testing.assert_allclose(wts.cpu().numpy(), o_w, rtol=2e-6, atol=1e-7)
        want = oslots.resolve(tab, o_ids[0].tolist())
        n = int(nm.item())
        assert out_slot.tolist() == want[0] and fs[:n].tolist() == want[1]
        assert fe[:n].tolist() == want[2]
    so, se, st, stp = tab.arrays()
    assert np.array_equal(slot_of.cpu().numpy(), so) and np.array_equal(stamp.cpu().numpy(), st)
    assert int(step.item()) == int(stp)


@pytest.mark.parametrize("E,H,T", [(320, 1056, 100), (256, 2048, 64), (40, 96, 65)])
def test_router_logits_matrix_cores_equal_vector_kernel(lib, dev, E, H, T):
    """From 64 tokens the logits run on the float64 matrix cores: the same
    logits, ids and weights as the vector kernel (the same call cut into
    pieces of fewer than 64 tokens), with a bias, ragged expert and token
    tiles, and the oracle's ids."""
    g = torch.Generator(device="cpu").manual_seed(E + H + T)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn((E, H), generator=g) * 0.02).to(torch.bfloat16).to(dev)
    bias = (torch.randn(E, generator=g) * 0.01).to(dev)
    K = 8
    out = [torch.empty((T, E), device=dev), torch.empty((T, K), dtype=torch.int32, device=dev),
           torch.empty((T, K), device=dev)]
    say(f"router matrix cores: E={E} H={H} T={T}")
    lib.router_topk(x, w, bias, K, out[0], out[1], out[2])
    ref = [torch.empty_like(t) for t in out]
    for t0 in range(0, T, 40):                    # pieces of at most 40 tokens
        t1 = min(T, t0 + 40)
        parts = [r[t0:t1] for r in ref]
        lib.router_topk(x[t0:t1], w, bias, K, *parts)
    torch.cuda.synchronize()
    for a, b, name in zip(out, ref, ("logits", "ids", "weights")):
        assert torch.equal(a, b), name
    o_ids, _, _ = orouter.route(x.float().cpu().numpy(), w.float().cpu().numpy(), K,
                                bias=bias.cpu().numpy())
    assert np.array_equal(out[1].cpu().numpy(), o_ids)
