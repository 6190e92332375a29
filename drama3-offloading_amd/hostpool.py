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
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

import hipfetch


@dataclass(frozen=True)
class RecordLayout:
    hidden: int = 2048
    inter: int = 512

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
        strided views along the expert axis."""
        n = rec.shape[0]
        H, I = self.hidden, self.inter
        w13 = rec[:, :self.off_w2].view(torch.float8_e4m3fn).view(n, 2 * I, H)
        w2 = rec[:, self.off_w2:self.off_s13].view(torch.float8_e4m3fn).view(n, H, I)
        s13 = rec[:, self.off_s13:self.off_s2].view(torch.float32).view(n, 2 * I // 128, H // 128)
        s2 = rec[:, self.off_s2:self.payload_bytes].view(torch.float32).view(n, H // 128, I // 128)
        return w13, s13, w2, s2

    def pack(self, w13: torch.Tensor, s13: torch.Tensor, w2: torch.Tensor,
             s2: torch.Tensor) -> torch.Tensor:
        """Dense per-buffer tensors [n, ...] -> packed uint8 records [n, record_bytes]."""
        n = w13.shape[0]
        rec = torch.zeros((n, self.record_bytes), dtype=torch.uint8, device=w13.device)
        rec[:, :self.off_w2] = w13.reshape(n, -1).view(torch.uint8)
        rec[:, self.off_w2:self.off_s13] = w2.reshape(n, -1).view(torch.uint8)
        rec[:, self.off_s13:self.off_s2] = s13.reshape(n, -1).contiguous().view(torch.uint8)
        rec[:, self.off_s2:self.payload_bytes] = s2.reshape(n, -1).contiguous().view(torch.uint8)
        return rec


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
        self.ptr = self.lib.host_alloc(self.nbytes, noncoherent=noncoherent)
        self.dev_ptr = self.lib.device_ptr_of(self.ptr)
        buf = (ctypes.c_uint8 * self.nbytes).from_address(self.ptr)
        self.array = np.ctypeslib.as_array(buf).reshape(n_experts, layout.record_bytes)
        self.tensor = torch.from_numpy(self.array)          # CPU view, no copy

    def write(self, first: int, records: torch.Tensor) -> None:
        """Copy packed records (any device) into experts first, first+1, ..."""
        n = records.shape[0]
        self.tensor[first:first + n].copy_(records)

    def fetch_pair(self, cache: torch.Tensor):
        """(src device address, dst address, bytes per record) for moe_fetch."""
        return (self.dev_ptr, cache.data_ptr(), self.layout.record_bytes)

    def close(self) -> None:
        if self.ptr:
            self.tensor = None
            self.array = None
            self.lib.host_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:                                     # noqa: BLE001
            pass
