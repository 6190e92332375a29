"""The CPU baseline bench.py times (oracle/cpu_moe.py, the reference's
dequantise-then-matmul path, notes/13-non-ada-gpus.md:37-53) computes what it
claims: on Drama-3-layout packed records its MoE equals oracle.moe's float64
W8A16 forward within bf16 rounding, and its decode step equals a float64
composition of stub matmul, router, experts and residual."""
import numpy as np
import torch

from oracle import cpu_moe
from oracle import moe as omoe

E, H, I, K = 16, 2048, 512, 8


def _pool(seed):
    import hostpool
    import synth
    parts = [synth.expert_tensors(seed, 0, e, H, I) for e in range(E)]
    w13, s13, w2, s2 = (torch.stack(t) for t in zip(*parts))
    rec = hostpool.DRAMA3.pack(w13, s13, w2, s2)
    return rec, (w13.numpy(), s13.numpy(), w2.numpy(), s2.numpy())


def test_moe_forward_cpu_equals_float64_w8a16_on_packed_records():
    import hostpool
    rec, dense = _pool(3)
    rng = np.random.default_rng(0)
    T = 3
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32))
    ids = torch.from_numpy(np.stack([rng.choice(E, K, replace=False) for _ in range(T)]))
    w = torch.from_numpy(rng.random((T, K)).astype(np.float32))
    w = w / w.sum(-1, keepdim=True)
    got = cpu_moe.moe_forward_cpu(x, ids, w, rec, hostpool.DRAMA3).numpy()
    want = omoe.forward_w8a16(x.numpy(), ids.numpy(), w.numpy().astype(np.float64), *dense)
    assert np.abs(got - want).max() <= 2 ** -8 * np.abs(want).max()
    # a record read with the scales of the wrong half lands far outside that bar
    bad = rec.clone()
    off = hostpool.DRAMA3.off_s13
    bad[:, off:off + 256], bad[:, off + 256:off + 512] = rec[:, off + 256:off + 512], rec[:, off:off + 256]
    wrong = cpu_moe.moe_forward_cpu(x, ids, w, bad, hostpool.DRAMA3).numpy()
    assert np.abs(wrong - want).max() > 0.05 * np.abs(want).max()
    # and so does a tile-ordered record read as row-major
    rows = hostpool.RecordLayout(H, I, tiled=False)
    wrong = cpu_moe.moe_forward_cpu(x, ids, w, rec, rows).numpy()
    assert np.abs(wrong - want).max() > 0.05 * np.abs(want).max()


def test_decode_step_cpu_equals_float64_composition():
    import hostpool
    rec, dense = _pool(4)
    rng = np.random.default_rng(1)
    L = 2
    x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32))
    w_stub = torch.from_numpy((rng.standard_normal((L, H, H)) / np.sqrt(H)).astype(np.float32))
    gate = torch.from_numpy((rng.standard_normal((L, E, H)) * 0.02).astype(np.float32))
    bias = torch.from_numpy(rng.gumbel(size=(L, E)).astype(np.float32))
    got = cpu_moe.decode_step_cpu(x, w_stub, gate, bias, rec[None].expand(L, -1, -1),
                                  hostpool.DRAMA3, top_k=K).numpy()
    xv = x.numpy().astype(np.float64)
    for l in range(L):
        h = xv @ w_stub[l].numpy().astype(np.float64).T
        logits = h @ gate[l].numpy().astype(np.float64).T + bias[l].numpy()
        ids = np.argsort(-logits[0], kind="stable")[:K]
        sel = logits[0, ids]
        wts = np.exp(sel - sel.max())
        wts /= wts.sum()
        y = omoe.forward_w8a16(h, ids[None], wts[None], *dense)
        xv = h + y.astype(np.float64)
    assert np.abs(got - xv).max() <= 2 ** -7 * np.abs(xv).max()
