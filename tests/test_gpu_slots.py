"""Device slot table on the GPU, bit-exact against the oracle restatement of
bin/devcache.py:45-98 over the reference's recorded router traces."""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import slots

pytestmark = pytest.mark.gpu


def _tables(lib, dev, E, C, n=1):
    tabs = []
    for _ in range(n):
        t = dict(slot_of=torch.empty(E, dtype=torch.int32, device=dev),
                 slot_expert=torch.empty(C, dtype=torch.int32, device=dev),
                 stamp=torch.empty(C, dtype=torch.int64, device=dev),
                 step=torch.empty(1, dtype=torch.int64, device=dev),
                 stats=torch.zeros(2, dtype=torch.int64, device=dev))
        lib.slots_init(t["slot_of"], t["slot_expert"], t["stamp"], t["step"])
        tabs.append(t)
    return tabs


def _same(t, o: slots.SlotTable):
    so, se, st, step = o.arrays()
    return (np.array_equal(t["slot_of"].cpu().numpy(), so)
            and np.array_equal(t["slot_expert"].cpu().numpy(), se)
            and np.array_equal(t["stamp"].cpu().numpy(), st)
            and int(t["step"].item()) == int(step))


def test_init_matches_reference_layout(lib, dev):
    (t,) = _tables(lib, dev, 256, 64)
    assert _same(t, slots.SlotTable.fresh(256, 64))


def test_hand_worked_sequence(lib, dev):
    (t,) = _tables(lib, dev, 8, 4)
    o = slots.SlotTable.fresh(8, 4)
    out = torch.zeros(2, dtype=torch.int32, device=dev)
    fs = torch.zeros(2, dtype=torch.int32, device=dev)
    fe = torch.zeros(2, dtype=torch.int32, device=dev)
    nm = torch.zeros(1, dtype=torch.int32, device=dev)
    for ids in ([0, 1], [2, 3], [4], [1, 5], [6, 6]):
        want = slots.resolve(o, ids)
        d = torch.tensor(ids, dtype=torch.int32, device=dev)
        lib.resolve_slots(d, t["slot_of"], t["slot_expert"], t["stamp"], t["step"], out, fs, fe,
                          nm, t["stats"])
        n = int(nm.item())
        assert out[:len(ids)].tolist() == want[0]
        assert fs[:n].tolist() == want[1] and fe[:n].tolist() == want[2]
        assert _same(t, o)


@pytest.mark.parametrize("name,cap", [("trace", 64), ("t512", 69), ("t512", 113),
                                      ("direct", 61), ("direct", 300)])
def test_reference_trace_bit_exact(lib, dev, traces, name, cap):
    layers = traces[f"{name}_decode_layer"].astype(np.int64)
    ids = traces[f"{name}_decode_ids"].astype(np.int32)
    N = len(layers)
    say(f"slots: {name} trace, {N} steps, cap {cap}")
    tabs = _tables(lib, dev, 256, cap, 40)
    d_ids = torch.from_numpy(ids).to(dev)
    out = torch.zeros((N, 8), dtype=torch.int32, device=dev)
    fs = torch.full((N, 8), -9, dtype=torch.int32, device=dev)
    fe = torch.full((N, 8), -9, dtype=torch.int32, device=dev)
    nm = torch.zeros((N, 1), dtype=torch.int32, device=dev)
    for i in range(N):
        t = tabs[layers[i]]
        lib.resolve_slots(d_ids[i], t["slot_of"], t["slot_expert"], t["stamp"], t["step"],
                          out[i], fs[i], fe[i], nm[i], t["stats"])
    torch.cuda.synchronize()
    o_tabs = [slots.SlotTable.fresh(256, cap) for _ in range(40)]
    out_h, fs_h, fe_h, nm_h = out.cpu().numpy(), fs.cpu().numpy(), fe.cpu().numpy(), nm.cpu().numpy()
    hits = np.zeros(40, np.int64)
    misses = np.zeros(40, np.int64)
    for i in range(N):
        o, f_s, f_e = slots.resolve(o_tabs[layers[i]], ids[i].tolist())
        n = len(f_s)
        assert out_h[i].tolist() == o, f"step {i}"
        assert nm_h[i, 0] == n and fs_h[i, :n].tolist() == f_s and fe_h[i, :n].tolist() == f_e
        hits[layers[i]] += 8 - n
        misses[layers[i]] += n
    for l in range(40):
        assert _same(tabs[l], o_tabs[l]), f"layer {l}"
        assert tabs[l]["stats"].tolist() == [hits[l], misses[l]]


@pytest.mark.parametrize("cap,E,K", [(1500, 4096, 16), (700, 1000, 8), (4096, 4096, 8), (7, 20, 3)])
def test_random_streams_all_capacity_paths(lib, dev, cap, E, K):
    rng = np.random.default_rng(cap)
    (t,) = _tables(lib, dev, E, cap)
    o = slots.SlotTable.fresh(E, cap)
    out = torch.zeros(K, dtype=torch.int32, device=dev)
    fs = torch.zeros(K, dtype=torch.int32, device=dev)
    fe = torch.zeros(K, dtype=torch.int32, device=dev)
    nm = torch.zeros(1, dtype=torch.int32, device=dev)
    say(f"slots: random cap {cap} E {E} K {K}")
    for step in range(300):
        ids = rng.choice(E, size=K, replace=False).astype(np.int64)
        d = torch.from_numpy(ids).to(dev)                       # int64 ids path
        lib.resolve_slots(d, t["slot_of"], t["slot_expert"], t["stamp"], t["step"], out, fs, fe,
                          nm, None)
        want = slots.resolve(o, ids.tolist())
        if step % 37 == 0 or step == 299:
            torch.cuda.synchronize()
            assert out.tolist() == want[0]
            assert _same(t, o)
    torch.cuda.synchronize()
    assert _same(t, o)


def test_out_of_range_id_is_reported_not_indexed(lib, dev):
    (t,) = _tables(lib, dev, 16, 4)
    out = torch.zeros(3, dtype=torch.int32, device=dev)
    fs = torch.zeros(3, dtype=torch.int32, device=dev)
    fe = torch.zeros(3, dtype=torch.int32, device=dev)
    nm = torch.zeros(1, dtype=torch.int32, device=dev)
    d = torch.tensor([3, 99, -1], dtype=torch.int32, device=dev)
    lib.resolve_slots(d, t["slot_of"], t["slot_expert"], t["stamp"], t["step"], out, fs, fe, nm,
                      None)
    torch.cuda.synchronize()
    assert out.tolist() == [0, -1, -1] and int(nm.item()) == 1
