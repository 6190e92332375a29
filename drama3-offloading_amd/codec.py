"""Entropy-coded host pools: the same expert records, fewer bytes over the
host link, decoded on the GPU into byte-exact cache slots.

The decode step with experts offloaded is bound by the host link: at ~60 %
hit it spends most of its time moving records from page-locked host memory.
A record's fp8 weights are block-scaled e4m3 bytes whose exponent nibble
takes few values, so a record codes to about 84 % of its size losslessly
(format and kernel in csrc/codec.hip).  A CodedPool holds one layer's records
that way; `fetch` is the coded counterpart of moe_fetch (same job lists, read
on the device, capturable), and the cache slots it fills are identical to
those moe_fetch fills from the raw pool.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

import hipfetch
from hostpool import RecordLayout

BLOCK = 8192          # fp8 bytes per coded block
MAX_LEN = 6           # longest exponent code, bits (two codes in the 12-bit table)
DEFAULT_WORKGROUPS = 32      # of 4 waves; 24-32 measured best for 1-8 record launches


def code_lengths(hist, max_len: int = MAX_LEN) -> np.ndarray:
    """Length-limited Huffman code lengths for the 16 exponent values by
    package-merge; every value gets a code (its count plus one)."""
    w = [int(h) + 1 for h in hist]
    n = len(w)
    leaves = sorted(((w[s], (s,)) for s in range(n)), key=lambda t: t[0])
    merged = leaves
    for _ in range(max_len - 1):
        pkg = [(merged[i][0] + merged[i + 1][0], merged[i][1] + merged[i + 1][1])
               for i in range(0, len(merged) - 1, 2)]
        merged = sorted(leaves + pkg, key=lambda t: t[0])
    ln = np.zeros(n, dtype=np.uint8)
    for _, syms in merged[:2 * n - 2]:
        for s in syms:
            ln[s] += 1
    return ln


class CodedPool:
    """One layer's records (uint8 [n, record_bytes], host), entropy-coded into
    one page-locked, device-mapped region, plus the device-resident index
    (record offsets, block offsets) and decode table the fetch kernel reads.

    layout: a RecordLayout (the packed record: its fp8 part is coded, the
    block scales after it are kept raw), or an int: the leading bytes of each
    record to code (e.g. the whole record of one expert's w13 buffer).
    lengths: code lengths to use (default: from this layer's own histogram).
    scratch: optional uint8 host buffer of at least codec_bound * n bytes,
    reused across layers."""

    def __init__(self, records: np.ndarray, layout: RecordLayout | int, device, lengths=None,
                 threads: int = 8, scratch: np.ndarray | None = None, noncoherent: bool = False):
        self.lib = lib = hipfetch.require()
        self.layout = layout if isinstance(layout, RecordLayout) else None
        n, rb = records.shape
        if self.layout is not None and rb != layout.record_bytes:
            raise ValueError("records do not match the layout")
        self.n = n
        self.record_bytes = rb
        self.fp8_bytes = layout.off_s13 if self.layout is not None else int(layout)
        if not 0 < self.fp8_bytes <= rb:
            raise ValueError(f"{self.fp8_bytes} coded bytes of a {rb}-byte record")
        if self.fp8_bytes % BLOCK:
            raise ValueError(f"fp8 part of {self.fp8_bytes} bytes is not a multiple of {BLOCK}")
        if lengths is None:
            lengths = code_lengths(lib.codec_histogram(records, self.fp8_bytes, threads))
        self.lengths = np.asarray(lengths, dtype=np.uint8)
        need = lib.codec_bound(rb, self.fp8_bytes) * n
        if scratch is None or scratch.nbytes < need:
            scratch = np.empty(need, dtype=np.uint8)
        used, rec_off, blk_off = lib.codec_encode(records, self.fp8_bytes, self.lengths,
                                                  scratch[:need], threads)
        self.coded_bytes = used
        self.raw_bytes = n * rb
        self.ptr, self._host = lib.host_buffer(used, noncoherent=noncoherent)
        ctypes.memmove(self.ptr, scratch.ctypes.data, used)
        self.dev_ptr = lib.device_ptr_of(self.ptr)
        self.rec_off = torch.from_numpy(rec_off).to(device)
        self.blk_off = torch.from_numpy(blk_off).to(device)
        self.lut = torch.from_numpy(lib.codec_table(self.lengths).view(np.int16)).to(device)

    @property
    def ratio(self) -> float:
        return self.coded_bytes / self.raw_bytes

    def fetch(self, cache: torch.Tensor, fetch_expert, fetch_slot, nmiss, max_jobs: int,
              workgroups: int = DEFAULT_WORKGROUPS) -> None:
        """Decode records fetch_expert[j] into cache slots fetch_slot[j],
        j < nmiss[0] (all read on the device)."""
        self.lib.fetch_coded(self.dev_ptr, self.rec_off, self.blk_off, self.record_bytes,
                             self.fp8_bytes, self.lut, fetch_expert, fetch_slot, nmiss, max_jobs,
                             cache, workgroups)

    def close(self) -> None:
        """Free the coded bytes (device addresses taken from the pool, such
        as a captured graph's, are the caller's to retire first)."""
        self._host = None
        self.ptr = 0
        self.dev_ptr = 0
