"""Host-pool loader from safetensors shards (CPU).

1. Against the reference's recorded checkpoint headers (layers 0 and 39 of
   notes/drama3-safetensors-headers.json.gz, committed as a fixture): every
   routed expert of a layer is found with the dtypes and shapes the record
   layout expects, and its six tensors fill exactly one 3,146,496-byte
   record.
2. Against synthetic shards written by the safetensors library with the
   checkpoint's tensor names: records equal hostpool.RecordLayout.pack of the
   same tensors byte for byte, and the reference-layout buffers equal the
   tensors; wrong dtypes and missing tensors are refused."""
import gzip
import json

import numpy as np
import pytest
import torch

from conftest import GOLDEN


def _fixture_index():
    import loader
    fx = json.load(gzip.open(GOLDEN / "drama3_mlp_headers.json.gz"))
    entries = fx["entries"]
    starts = {m["shard"]: 0 for m in entries.values()}
    return loader.ShardIndex(None, entries, starts), entries


def test_plan_matches_reference_checkpoint_layout():
    import loader
    from hostpool import DRAMA3
    index, entries = _fixture_index()
    for layer in (0, 39):
        assert index.n_experts(layer) == 256
        plan = loader.layer_plan(index, layer, DRAMA3)
        assert len(plan) == 256
        for rec in plan:
            assert sum(t.nbytes for t, _ in rec) == DRAMA3.record_bytes == 3_146_496
            assert DRAMA3.payload_bytes == DRAMA3.record_bytes
            offs = sorted((off, t.nbytes) for t, off in rec)
            for (o0, n0), (o1, _) in zip(offs, offs[1:]):
                assert o0 + n0 == o1                     # contiguous, no gaps or overlap
        gate = index.get(loader.ROUTER_GATE.format(layer=layer))
        assert gate.dtype == "BF16" and gate.shape == (256, 2048)
    for layer in (0, 39):
        for proj, shape in (("gate_proj", [512, 2048]), ("up_proj", [512, 2048]),
                            ("down_proj", [2048, 512])):
            m = entries[loader.SHARED.format(layer=layer, proj=proj)]
            assert m["dtype"] == "BF16" and m["shape"] == shape
        m = entries[loader.SHARED_GATE.format(layer=layer)]
        assert m["dtype"] == "BF16" and m["shape"] == [1, 2048]


def _write_shards(tmp_path, layers=2, E=6, H=256, I=128, seed=0):
    from safetensors.torch import save_file
    from loader import EXPERT
    g = torch.Generator().manual_seed(seed)
    # finite codes of magnitude < 2 with random signs (no NaN codes 0x7f / 0xff)
    f8 = lambda *s: (torch.randint(0, 0x40, s, generator=g, dtype=torch.uint8)          # noqa
                     | (torch.randint(0, 2, s, generator=g, dtype=torch.uint8) << 7)
                     ).view(torch.float8_e4m3fn)
    sc = lambda *s: torch.rand(s, generator=g) + 0.5                                                       # noqa
    tensors = {}
    for l in range(layers):
        for e in range(E):
            for proj, shape in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
                tensors[EXPERT.format(layer=l, expert=e, proj=proj, what="weight")] = f8(*shape)
                tensors[EXPERT.format(layer=l, expert=e, proj=proj, what="weight_scale_inv")] = \
                    sc(shape[0] // 128, shape[1] // 128)
        tensors[f"model.language_model.layers.{l}.mlp.gate.weight"] = torch.zeros((E, H),
                                                                                   dtype=torch.bfloat16)
        bf = lambda *s: torch.randn(s, generator=g).to(torch.bfloat16)               # noqa
        for proj, shape in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            tensors[f"model.language_model.layers.{l}.mlp.shared_expert.{proj}.weight"] = bf(*shape)
        tensors[f"model.language_model.layers.{l}.mlp.shared_expert_gate.weight"] = bf(1, H)
    names = sorted(tensors)
    half = len(names) // 2 + 3                   # split one layer's experts across both shards
    save_file({n: tensors[n] for n in names[:half]}, tmp_path / "model-00001-of-00002.safetensors")
    save_file({n: tensors[n] for n in names[half:]}, tmp_path / "model-00002-of-00002.safetensors")
    return tensors


def _expert(tensors, l, e, what):
    from loader import EXPERT
    return [tensors[EXPERT.format(layer=l, expert=e, proj=p, what=what)]
            for p in ("gate_proj", "up_proj", "down_proj")]


def test_records_from_shards_equal_packed_tensors(tmp_path):
    import loader
    from hostpool import RecordLayout
    tensors = _write_shards(tmp_path)
    lay = RecordLayout(256, 128)
    index = loader.ShardIndex.from_dir(tmp_path)
    assert index.n_experts(0) == 6 and index.n_experts(1) == 6
    for l in range(2):
        dst = np.zeros((6, lay.record_bytes), np.uint8)
        assert loader.fill_records(index, l, dst, lay, threads=3) == 6 * lay.payload_bytes
        for e in range(6):
            g, u, d = _expert(tensors, l, e, "weight")
            gs, us, ds = _expert(tensors, l, e, "weight_scale_inv")
            want = lay.pack(torch.cat([g, u])[None], torch.cat([gs, us])[None], d[None], ds[None])
            assert np.array_equal(dst[e], want[0].numpy()), f"layer {l} expert {e}"


def test_reference_layout_buffers_from_shards(tmp_path):
    import loader
    import moe
    tensors = _write_shards(tmp_path, seed=3)
    index = loader.ShardIndex.from_dir(tmp_path)
    m = moe.MoEExperts(6, 256, 128)
    loader.fill_expert_buffers(index, 1, m, threads=2)
    for e in range(6):
        g, u, d = _expert(tensors, 1, e, "weight")
        gs, us, ds = _expert(tensors, 1, e, "weight_scale_inv")
        assert torch.equal(m.w13_weight[e].view(torch.uint8), torch.cat([g, u]).view(torch.uint8))
        assert torch.equal(m.w2_weight[e].view(torch.uint8), d.view(torch.uint8))
        assert torch.equal(m.w13_scale_inv[e], torch.cat([gs, us]))
        assert torch.equal(m.w2_scale_inv[e], ds)


def test_wrong_dtype_and_missing_tensor_are_refused(tmp_path):
    import loader
    from hostpool import RecordLayout
    from safetensors.torch import save_file
    lay = RecordLayout(256, 128)
    t = {loader.EXPERT.format(layer=0, expert=0, proj="gate_proj", what="weight"):
         torch.zeros((128, 256), dtype=torch.bfloat16)}
    save_file(t, tmp_path / "a.safetensors")
    index = loader.ShardIndex.from_dir(tmp_path)
    with pytest.raises(ValueError, match="F8_E4M3"):
        loader.record_plan(index, 0, 0, lay)
    with pytest.raises(KeyError, match="layers.3"):
        loader.record_plan(index, 3, 0, lay)


def test_shared_expert_from_shards(tmp_path):
    import loader
    tensors = _write_shards(tmp_path, seed=5)
    index = loader.ShardIndex.from_dir(tmp_path)
    for l in range(2):
        got = loader.load_shared_expert(index, l)
        pre = f"model.language_model.layers.{l}.mlp."
        assert torch.equal(got["gate"], tensors[pre + "shared_expert.gate_proj.weight"])
        assert torch.equal(got["up"], tensors[pre + "shared_expert.up_proj.weight"])
        assert torch.equal(got["down"], tensors[pre + "shared_expert.down_proj.weight"])
        assert torch.equal(got["sgate"], tensors[pre + "shared_expert_gate.weight"].reshape(-1))
        assert got["gate"].shape == (128, 256) and got["sgate"].shape == (256,)
