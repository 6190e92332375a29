"""One page-locked region of packed expert records per layer.

The reference pins 4 tensors per layer, 160 separate power-of-two-rounded
allocations for 40 layers (bin/offload.py:664-699; the waste and the
scattered bases are noted at bin/bench_hostread.py:262-269).  Here a layer's
256 experts are one hipHostMalloc'd, device-mapped region of records

    record e = w13 (2I x H e4m3) | w2 (H x I e4m3) | s13 (2I/128 x H/128 f32)
               | s2 (H/128 x I/128 f32)

3,146,496 B each at Drama-3 shapes (2^8 * 3 * 17 * 241, so every record
starts 256-byte aligned), and a miss is ONE contiguous copy of one record.
The device cache holds records in the same layout, and the expert FFN reads
them in place through strided views (moe_expert_strides).

The two e4m3 matrices are stored in MFMA tile order (MOE_LAYOUT_TILES, see
to_tiles): each 16-row x 128-column block is 2 KiB laid out as the 64 lanes
of a wave load it, so every 16-byte load of the expert kernels reads 1 KiB
contiguous.  The scales are row-major.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

import hipfetch


def _order(t, perm):
    """permute for torch tensors, transpose for numpy arrays, made contiguous."""
    if isinstance(t, np.ndarray):
        return np.ascontiguousarray(t.transpose(perm))
    return t.permute(*perm).contiguous()


def to_tiles(w):
    """[..., R, K] row-major e4m3 bytes (R % 16 == 0, K % 128 == 0; torch or
    numpy, any 1-byte dtype) -> the same shape in MFMA tile order: row group
    g = row // 16, then K-block b = col // 128, then 1 KiB half h, then
    16-byte unit 16q + r, then byte i, where row = 16g + r and col = 128b +
    32q + 16h + i.  Unit 16q + r of half h is what lane 16q + r of a wave
    loads for the 16x16x128 MFMA's A operand (row r, reduction indices
    32q + 16h ..)."""
    *lead, R, K = w.shape
    n = len(lead)
    t = w.reshape(*lead, R // 16, 16, K // 128, 4, 2, 16)            # g r b q h i
    perm = list(range(n)) + [n + 0, n + 2, n + 4, n + 3, n + 1, n + 5]   # g b h q r i
    return _order(t, perm).reshape(*lead, R, K)


def from_tiles(w):
    """Inverse of to_tiles."""
    *lead, R, K = w.shape
    n = len(lead)
    t = w.reshape(*lead, R // 16, K // 128, 2, 4, 16, 16)            # g b h q r i
    perm = list(range(n)) + [n + 0, n + 4, n + 1, n + 3, n + 2, n + 5]   # g r b q h i
    return _order(t, perm).reshape(*lead, R, K)


@dataclass(frozen=True)
class RecordLayout:
    hidden: int = 2048
    inter: int = 512
    tiled: bool = True          # w13/w2 in MFMA tile order (else row-major)

    @property
    def code(self) -> int:
        """moe_expert_strides.layout of this layout's records."""
        return hipfetch.LAYOUT_TILES if self.tiled else hipfetch.LAYOUT_ROWS

    @property
    def w13_bytes(self) -> int:
        return 2 * self.inter * self.hidden

    @property
    def w2_bytes(self) -> int:
        return self.hidden * self.inter

    @property
    def s13_bytes(self) -> int:
        return (2 * self.inter // 128) * (self.hidden // 128) * 4

    @property
    def s2_bytes(self) -> int:
        return (self.hidden // 128) * (self.inter // 128) * 4

    @property
    def off_w2(self) -> int:
        return self.w13_bytes

    @property
    def off_s13(self) -> int:
        return self.w13_bytes + self.w2_bytes

    @property
    def off_s2(self) -> int:
        return self.off_s13 + self.s13_bytes

    @property
    def payload_bytes(self) -> int:
        return self.off_s2 + self.s2_bytes

    @property
    def record_bytes(self) -> int:
        """Payload rounded up to 256 bytes, so every record of a pool starts
        256-byte aligned (the kernels' 16-byte loads need it); Drama-3's
        3,146,496-byte record needs no padding."""
        return (self.payload_bytes + 255) // 256 * 256

    def views(self, rec: torch.Tensor):
        """uint8 [n, record_bytes] -> (w13 e4m3 [n,2I,H], s13 f32, w2 e4m3 [n,H,I], s2 f32),
        strided views along the expert axis.  w13/w2 hold the record's bytes
        as stored: pass `layout=self.code` to the expert FFN."""
        n = rec.shape[0]
        H, I = self.hidden, self.inter
        w13 = rec[:, :self.off_w2].view(torch.float8_e4m3fn).view(n, 2 * I, H)
        w2 = rec[:, self.off_w2:self.off_s13].view(torch.float8_e4m3fn).view(n, H, I)
        s13 = rec[:, self.off_s13:self.off_s2].view(torch.float32).view(n, 2 * I // 128, H // 128)
        s2 = rec[:, self.off_s2:self.payload_bytes].view(torch.float32).view(n, H // 128, I // 128)
        return w13, s13, w2, s2

    def pack(self, w13: torch.Tensor, s13: torch.Tensor, w2: torch.Tensor,
             s2: torch.Tensor) -> torch.Tensor:
        """Dense row-major per-buffer tensors [n, ...] (the checkpoint's
        layout) -> packed uint8 records [n, record_bytes]."""
        n = w13.shape[0]
        rec = torch.zeros((n, self.record_bytes), dtype=torch.uint8, device=w13.device)
        w13b, w2b = w13.view(torch.uint8), w2.view(torch.uint8)
        if self.tiled:
            w13b, w2b = to_tiles(w13b), to_tiles(w2b)
        rec[:, :self.off_w2] = w13b.reshape(n, -1)
        rec[:, self.off_w2:self.off_s13] = w2b.reshape(n, -1)
        rec[:, self.off_s13:self.off_s2] = s13.reshape(n, -1).contiguous().view(torch.uint8)
        rec[:, self.off_s2:self.payload_bytes] = s2.reshape(n, -1).contiguous().view(torch.uint8)
        return rec

    def unpack(self, rec):
        """Packed records [n, record_bytes] (torch or numpy uint8) -> dense
        row-major (w13 uint8 [n,2I,H], s13 f32, w2 uint8 [n,H,I], s2 f32),
        the inverse of pack; copies."""
        n = rec.shape[0]
        H, I = self.hidden, self.inter
        w13 = rec[:, :self.off_w2].reshape(n, 2 * I, H)
        w2 = rec[:, self.off_w2:self.off_s13].reshape(n, H, I)
        if self.tiled:
            w13, w2 = from_tiles(w13), from_tiles(w2)
        if isinstance(rec, np.ndarray):
            f32 = lambda b: np.ascontiguousarray(b).view(np.float32)
            w13, w2 = np.array(w13), np.array(w2)
        else:
            f32 = lambda b: b.contiguous().view(torch.float32)
            w13, w2 = w13.contiguous(), w2.contiguous()
        s13 = f32(rec[:, self.off_s13:self.off_s2]).reshape(n, 2 * I // 128, H // 128)
        s2 = f32(rec[:, self.off_s2:self.payload_bytes]).reshape(n, H // 128, I // 128)
        return w13, s13, w2, s2


DRAMA3 = RecordLayout()
assert DRAMA3.record_bytes == 3_146_496


class HostPool:
    """n_experts packed records in one page-locked, device-mapped region."""

    def __init__(self, n_experts: int, layout: RecordLayout = DRAMA3,
                 noncoherent: bool = False):
        self.lib = hipfetch.require()
        self.layout = layout
        self.n = n_experts
        self.nbytes = n_experts * layout.record_bytes
        # the memory lives as long as any view of it (self.array, self.tensor
        # or a slice taken from them)
        self.ptr, flat = self.lib.host_buffer(self.nbytes, noncoherent=noncoherent)
        self.dev_ptr = self.lib.device_ptr_of(self.ptr)
        self.array = flat.reshape(n_experts, layout.record_bytes)
        self.tensor = torch.from_numpy(self.array)          # CPU view, no copy

    def write(self, first: int, records: torch.Tensor) -> None:
        """Copy packed records (any device) into experts first, first+1, ..."""
        n = records.shape[0]
        self.tensor[first:first + n].copy_(records)

    def to_experts(self, experts, device, chunk: int = 64) -> None:
        """Fill an experts module's four host buffers (w13_weight [E, 2I, H],
        w13_scale_inv, w2_weight, w2_scale_inv: the reference's layout,
        row-major) with this pool's experts, unpacking `chunk` records at a
        time on `device`."""
        if experts.w13_weight.shape[0] != self.n:
            raise ValueError(f"{experts.w13_weight.shape[0]} experts in the module, "
                             f"{self.n} in the pool")
        for first in range(0, self.n, chunk):
            last = min(self.n, first + chunk)
            w13, s13, w2, s2 = self.layout.unpack(self.tensor[first:last].to(device))
            experts.w13_weight.view(torch.uint8)[first:last].copy_(w13)
            experts.w13_scale_inv[first:last].copy_(s13)
            experts.w2_weight.view(torch.uint8)[first:last].copy_(w2)
            experts.w2_scale_inv[first:last].copy_(s2)

    def fetch_pair(self, cache: torch.Tensor):
        """(src device address, dst address, bytes per record) for moe_fetch."""
        return (self.dev_ptr, cache.data_ptr(), self.layout.record_bytes)

    def close(self) -> None:
        """Drop the pool's views: the memory is freed now unless a slice of
        it is still held elsewhere, then when that goes.  Device addresses
        taken from the pool (dev_ptr, fetch_pair, a captured graph's) are
        the caller's to retire first."""
        self.tensor = None
        self.array = None
        self.ptr = 0
        self.dev_ptr = 0
