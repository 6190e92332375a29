"""Host expert pools straight from the model's safetensors shards.

The reference loads the whole model through upstream's loader, moves each
layer's experts to the CPU (bin/offload.py:111-134) and page-locks them as
four tensors per layer, 160 separate allocations (bin/offload.py:664-699).
Here the routed experts go directly from the checkpoint files into one
page-locked region of packed records per layer (hostpool.HostPool):

    record e = gate_proj | up_proj            (w13, 2I x H e4m3, gate rows first)
             | down_proj                      (w2, H x I e4m3)
             | gate scale_inv | up scale_inv  (s13, 2I/128 x H/128 f32)
             | down scale_inv                 (s2, H/128 x I/128 f32)

The checkpoint stores every expert as six tensors,
`model.language_model.layers.{l}.mlp.experts.{e}.{gate,up,down}_proj.weight`
(F8_E4M3) and `...weight_scale_inv` (F32), spread over the shards
(notes/drama3-safetensors-headers.json.gz).  A safetensors file is an 8-byte
little-endian header length, a JSON header of {name: dtype, shape,
data_offsets}, then the data; the loader memory-maps each shard and copies
byte ranges, so nothing is converted and the host never holds a second copy.
Copies run on a thread pool (numpy releases the GIL while copying).
"""
from __future__ import annotations

import json
import struct
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from hostpool import RecordLayout, to_tiles

EXPERT = "model.language_model.layers.{layer}.mlp.experts.{expert}.{proj}.{what}"
ROUTER_GATE = "model.language_model.layers.{layer}.mlp.gate.weight"
SHARED = "model.language_model.layers.{layer}.mlp.shared_expert.{proj}.weight"
SHARED_GATE = "model.language_model.layers.{layer}.mlp.shared_expert_gate.weight"
_DTYPE_BYTES = {"F8_E4M3": 1, "BF16": 2, "F16": 2, "F32": 4}


@dataclass(frozen=True)
class TensorEntry:
    shard: str          # shard file name
    dtype: str
    shape: tuple
    start: int          # absolute byte offset in the shard file
    nbytes: int


def read_header(path: Path) -> tuple[dict, int]:
    """(header dict, byte offset of the data section) of one safetensors file."""
    with open(path, "rb") as f:
        (n,) = struct.unpack("<Q", f.read(8))
        return json.loads(f.read(n)), 8 + n


class ShardIndex:
    """Where every tensor of a checkpoint lives.

    entries: {name: {"shard", "dtype", "shape", "data_offsets"}} plus each
    shard's data offset, either read from the files (from_dir) or given
    (e.g. a recorded header)."""

    def __init__(self, root: Path | None, entries: dict, data_start: dict[str, int]):
        self.root = Path(root) if root is not None else None
        self.tensors: dict[str, TensorEntry] = {}
        for name, m in entries.items():
            a, b = m["data_offsets"]
            t = TensorEntry(m["shard"], m["dtype"], tuple(m["shape"]), data_start[m["shard"]] + a,
                            b - a)
            want = int(np.prod(t.shape)) * _DTYPE_BYTES.get(t.dtype, 0)
            if want != t.nbytes:
                raise ValueError(f"{name}: {t.nbytes} bytes for {t.dtype}{list(t.shape)}")
            self.tensors[name] = t

    @classmethod
    def from_dir(cls, root) -> "ShardIndex":
        root = Path(root)
        entries, starts = {}, {}
        for path in sorted(root.glob("*.safetensors")):
            hdr, start = read_header(path)
            starts[path.name] = start
            for name, m in hdr.items():
                if name != "__metadata__":
                    entries[name] = {"shard": path.name, **m}
        if not entries:
            raise FileNotFoundError(f"no safetensors shards under {root}")
        return cls(root, entries, starts)

    def get(self, name: str) -> TensorEntry:
        t = self.tensors.get(name)
        if t is None:
            raise KeyError(f"checkpoint has no tensor {name!r}")
        return t

    def n_experts(self, layer: int) -> int:
        n = 0
        while EXPERT.format(layer=layer, expert=n, proj="gate_proj", what="weight") in self.tensors:
            n += 1
        return n


def _expect(t: TensorEntry, name: str, dtype: str, shape: tuple) -> None:
    if t.dtype != dtype or t.shape != shape:
        raise ValueError(f"{name}: expected {dtype}{list(shape)}, checkpoint has "
                         f"{t.dtype}{list(t.shape)}")


def record_plan(index: ShardIndex, layer: int, expert: int, layout: RecordLayout):
    """[(entry, offset in the record)] for the six tensors of one expert, in
    record order; checks every dtype and shape against the layout."""
    H, I = layout.hidden, layout.inter
    spec = [("gate_proj", "weight", "F8_E4M3", (I, H), 0),
            ("up_proj", "weight", "F8_E4M3", (I, H), I * H),
            ("down_proj", "weight", "F8_E4M3", (H, I), layout.off_w2),
            ("gate_proj", "weight_scale_inv", "F32", (I // 128, H // 128), layout.off_s13),
            ("up_proj", "weight_scale_inv", "F32", (I // 128, H // 128),
             layout.off_s13 + layout.s13_bytes // 2),
            ("down_proj", "weight_scale_inv", "F32", (H // 128, I // 128), layout.off_s2)]
    plan = []
    for proj, what, dtype, shape, off in spec:
        name = EXPERT.format(layer=layer, expert=expert, proj=proj, what=what)
        t = index.get(name)
        _expect(t, name, dtype, shape)
        plan.append((t, off))
    if sum(t.nbytes for t, _ in plan) != layout.payload_bytes:
        raise ValueError("expert tensors do not fill one record")
    return plan


def layer_plan(index: ShardIndex, layer: int, layout: RecordLayout, n_experts: int | None = None):
    n = index.n_experts(layer) if n_experts is None else n_experts
    if n == 0:
        raise KeyError(f"no routed experts for layer {layer}")
    return [record_plan(index, layer, e, layout) for e in range(n)]


class _Maps:
    """Read-only memory maps of the shards, opened on first use."""

    def __init__(self, root: Path):
        self.root = root
        self.maps: dict[str, np.memmap] = {}

    def __call__(self, shard: str) -> np.memmap:
        m = self.maps.get(shard)
        if m is None:
            m = np.memmap(self.root / shard, dtype=np.uint8, mode="r")
            self.maps[shard] = m
        return m


def fill_records(index: ShardIndex, layer: int, dst: np.ndarray, layout: RecordLayout,
                 threads: int = 8) -> int:
    """Copy layer `layer`'s experts into dst, a uint8 array [n_experts,
    record_bytes] (a HostPool's .array).  Returns the payload bytes copied."""
    if index.root is None:
        raise ValueError("index has no shard directory to read from")
    plan = layer_plan(index, layer, layout, dst.shape[0])
    maps = _Maps(index.root)

    def one(e: int) -> int:
        row = dst[e]
        for t, off in plan[e]:
            src = maps(t.shard)[t.start:t.start + t.nbytes]
            if layout.tiled and t.dtype == "F8_E4M3":
                # gate, up and down each tile on their own: gate's and up's
                # 16-row groups do not mix, so gate | up tiled is w13 tiled
                src = to_tiles(src.reshape(t.shape)).reshape(-1)
            row[off:off + t.nbytes] = src
        row[layout.payload_bytes:] = 0          # alignment padding, if any
        return layout.payload_bytes

    with ThreadPoolExecutor(max_workers=max(1, threads)) as ex:
        return sum(ex.map(one, range(dst.shape[0])))


def load_host_pools(root, layers, layout: RecordLayout, threads: int = 8, noncoherent=False):
    """One page-locked HostPool per layer in `layers`, filled from the shards
    under `root`.  Returns (pools, bytes copied)."""
    from hostpool import HostPool
    index = ShardIndex.from_dir(root)
    pools, total = [], 0
    try:
        for layer in layers:
            pool = HostPool(index.n_experts(layer), layout, noncoherent=noncoherent)
            pools.append(pool)
            total += fill_records(index, layer, pool.array, layout, threads)
    except Exception:
        for p in pools:
            p.close()
        raise
    return pools, total


def fill_expert_buffers(index: ShardIndex, layer: int, experts, threads: int = 8) -> None:
    """The reference's layout instead: an experts module's four host buffers
    (w13_weight [E, 2I, H], w2_weight, w13_scale_inv, w2_scale_inv, CPU,
    ideally page-locked) filled from the shards."""
    import torch
    H = experts.w13_weight.shape[2]
    I = experts.w2_weight.shape[2]
    layout = RecordLayout(H, I)
    n = experts.w13_weight.shape[0]
    plan = layer_plan(index, layer, layout, n)
    maps = _Maps(index.root)
    bufs = [experts.w13_weight.view(torch.uint8).numpy().reshape(n, -1),
            experts.w2_weight.view(torch.uint8).numpy().reshape(n, -1),
            experts.w13_scale_inv.numpy().view(np.uint8).reshape(n, -1),
            experts.w2_scale_inv.numpy().view(np.uint8).reshape(n, -1)]
    # record offset -> (buffer, offset inside the buffer's row)
    where = {0: (0, 0), I * H: (0, I * H), layout.off_w2: (1, 0), layout.off_s13: (2, 0),
             layout.off_s13 + layout.s13_bytes // 2: (2, layout.s13_bytes // 2),
             layout.off_s2: (3, 0)}

    def one(e: int) -> None:
        for t, off in plan[e]:
            b, o = where[off]
            bufs[b][e, o:o + t.nbytes] = maps(t.shard)[t.start:t.start + t.nbytes]

    with ThreadPoolExecutor(max_workers=max(1, threads)) as ex:
        list(ex.map(one, range(n)))


def load_shared_expert(index: ShardIndex, layer: int, device=None) -> dict:
    """The layer's gated shared expert as bf16 tensors, shaped as the shared
    expert kernels take them: {"gate": [Is, H], "up": [Is, H], "down": [H, Is],
    "sgate": [H]} (checkpoint tensors layers.N.mlp.shared_expert.*_proj.weight
    and layers.N.mlp.shared_expert_gate.weight [1, H], all BF16)."""
    import torch
    if index.root is None:
        raise ValueError("index has no shard directory to read from")
    names = {"gate": SHARED.format(layer=layer, proj="gate_proj"),
             "up": SHARED.format(layer=layer, proj="up_proj"),
             "down": SHARED.format(layer=layer, proj="down_proj"),
             "sgate": SHARED_GATE.format(layer=layer)}
    ent = {k: index.get(n) for k, n in names.items()}
    Is, H = ent["gate"].shape
    want = {"gate": (Is, H), "up": (Is, H), "down": (H, Is), "sgate": (1, H)}
    maps = _Maps(index.root)
    out = {}
    for k, t in ent.items():
        _expect(t, names[k], "BF16", want[k])
        raw = np.array(maps(t.shard)[t.start:t.start + t.nbytes])      # own copy
        v = torch.from_numpy(raw).view(torch.bfloat16).view(*t.shape)
        out[k] = v.reshape(-1) if k == "sgate" else v
    if device is not None:
        out = {k: v.to(device) for k, v in out.items()}
    return out
