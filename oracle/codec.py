"""The coded-record format, restated for checking (oracle, test
infrastructure).

A plain-Python encoder and decoder of the format the HIP library writes and
reads (drama3-offloading_amd/csrc/codec.hip); the reference stores records
raw (bin/offload.py:603, 3,146,496 B per expert), so the property that
matters is that decoding gives back exactly those bytes.  Written from the
format's definition, not from the library's code:

  fp8 block of 8192 bytes x ->
    nibble plane  4096 B: nibble byte m of lane l (symbols x[128l + 2m] and
                  x[128l + 2m + 1]) = nib(first) | nib(second) << 4, stored
                  at 16 * (64 * (m // 16) + l) + m % 16;
                  nib(v) = (v >> 7) << 3 | (v & 7)
    header        64 B:   byte l = byte length of stream l
    streams:      stream l = exponents (v >> 3) & 15 of x[128l:128l+128],
                  canonical Huffman codes (codes of one length consecutive,
                  shorter lengths first, symbols in increasing order within a
                  length), each code's bits emitted most significant first
                  into a bit sequence that fills bytes from bit 0 up; the
                  stream is padded with zero bits to a whole byte
    zero padding to a multiple of 16 bytes.
  A record: its blocks in order, then the bytes after the fp8 part raw;
  padded with zeros to a multiple of 256 bytes.
"""
from __future__ import annotations

import numpy as np

BLOCK = 8192
LANES = 64
PER_LANE = BLOCK // LANES
ALIGN = 16


def canonical(lengths):
    """{symbol: (code, length)}, codes as integers read most significant bit first."""
    out = {}
    code = 0
    for ln in range(1, max(int(v) for v in lengths) + 1):
        for s, l in enumerate(lengths):
            if int(l) == ln:
                out[s] = (code, ln)
                code += 1
        code <<= 1
    return out


def encode_block(x: np.ndarray, lengths) -> bytes:
    x = np.asarray(x, dtype=np.uint8)
    assert x.size == BLOCK
    nib = ((x >> 7) << 3) | (x & 7)
    pairs = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)      # [lane * 64 + m]
    plane = bytearray(BLOCK // 2)
    for lane in range(LANES):
        for m in range(PER_LANE // 2):
            plane[16 * (LANES * (m // 16) + lane) + m % 16] = pairs[lane * (PER_LANE // 2) + m]
    plane = bytes(plane)
    codes = canonical(lengths)
    header = bytearray()
    streams = bytearray()
    for lane in range(LANES):
        bits = []
        for v in x[lane * PER_LANE:(lane + 1) * PER_LANE]:
            c, ln = codes[(int(v) >> 3) & 15]
            bits.extend((c >> (ln - 1 - k)) & 1 for k in range(ln))
        while len(bits) % 8:
            bits.append(0)
        stream = bytes(sum(bits[i + k] << k for k in range(8)) for i in range(0, len(bits), 8))
        header.append(len(stream))
        streams.extend(stream)
    out = plane + bytes(header) + bytes(streams)
    return out + bytes(-len(out) % ALIGN)


def decode_block(blob: bytes, lengths) -> np.ndarray:
    codes = canonical(lengths)
    by_code = {(c, ln): s for s, (c, ln) in codes.items()}
    plane = np.frombuffer(blob[:BLOCK // 2], dtype=np.uint8)
    pairs = np.empty(BLOCK // 2, dtype=np.uint8)
    for lane in range(LANES):
        for m in range(PER_LANE // 2):
            pairs[lane * (PER_LANE // 2) + m] = plane[16 * (LANES * (m // 16) + lane) + m % 16]
    nib = np.empty(BLOCK, dtype=np.uint8)
    nib[0::2] = pairs & 15
    nib[1::2] = pairs >> 4
    header = blob[BLOCK // 2:BLOCK // 2 + LANES]
    pos = BLOCK // 2 + LANES
    out = np.empty(BLOCK, dtype=np.uint8)
    for lane in range(LANES):
        stream = blob[pos:pos + header[lane]]
        pos += header[lane]
        bits = [(b >> k) & 1 for b in stream for k in range(8)]
        i = 0
        for n in range(PER_LANE):
            c, ln = 0, 0
            while (c, ln) not in by_code:
                c = (c << 1) | bits[i]
                ln += 1
                i += 1
            e = by_code[(c, ln)]
            v = nib[lane * PER_LANE + n]
            out[lane * PER_LANE + n] = ((v >> 3) << 7) | (e << 3) | (v & 7)
    return out


def encode_record(rec: np.ndarray, fp8_bytes: int, lengths):
    """(coded bytes, block offsets [nblk + 1]) of one record."""
    rec = np.asarray(rec, dtype=np.uint8)
    parts, offs, o = [], [], 0
    for b in range(fp8_bytes // BLOCK):
        offs.append(o)
        blk = encode_block(rec[b * BLOCK:(b + 1) * BLOCK], lengths)
        parts.append(blk)
        o += len(blk)
    offs.append(o)
    data = b"".join(parts) + rec[fp8_bytes:].tobytes()
    return data + bytes(-len(data) % 256), offs


def decode_record(blob: bytes, offs, fp8_bytes: int, record_bytes: int, lengths) -> np.ndarray:
    nblk = fp8_bytes // BLOCK
    out = [decode_block(blob[offs[b]:offs[b + 1]], lengths) for b in range(nblk)]
    tail = np.frombuffer(blob[offs[nblk]:offs[nblk] + record_bytes - fp8_bytes], dtype=np.uint8)
    return np.concatenate(out + [tail])
