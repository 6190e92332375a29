"""OCP float8 e4m3fn codec and the block quantisation used by the experts.

Oracle (test infrastructure). Format facts:
  * e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa bits; no infinities;
    S.1111.111 is NaN; largest finite 448; smallest subnormal 2^-9.
  * The checkpoint stores experts as F8_E4M3 with F32 `weight_scale_inv`
    blocks of 128x128 (notes/drama3-safetensors-headers.json.gz: gate/up
    scale [4,16] for a [512,2048] weight, down scale [16,4] for [2048,512];
    notes/drama3-config.json quantization_config.weight_block_size).
  * Dequantisation is w = q * scale_inv[r // 128, c // 128] (upstream
    `dequantize_fp8_blocks`, described in notes/13-non-ada-gpus.md:43-53).
  * Activations are quantised dynamically (quantization_config
    activation_scheme "dynamic"): per token, per 128-wide group along the
    reduction axis, scale = amax / 448.  The reference only fixes "dynamic";
    the group width and the amax/448 rule are this build's stated contract
    (the common block-FP8 convention).  An all-zero group gets scale 0 and
    quantises to zeros; the reference notes that its kernel turns such a
    group into NaN (bin/offload.py:351-355) -- this contract does not.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0
_F32 = np.float32


def decode_table() -> np.ndarray:
    """float64 value of every e4m3fn code 0..255 (NaN for 0x7F / 0xFF)."""
    codes = np.arange(256, dtype=np.int64)
    sign = np.where(codes & 0x80, -1.0, 1.0)
    exp = (codes >> 3) & 0xF
    man = codes & 0x7
    sub = man.astype(np.float64) * 2.0 ** -9
    nor = (1.0 + man / 8.0) * np.exp2(exp.astype(np.float64) - 7.0)
    val = sign * np.where(exp == 0, sub, nor)
    val[(codes & 0x7F) == 0x7F] = np.nan
    return val


_DEC = decode_table()


def decode(q: np.ndarray) -> np.ndarray:
    """uint8 codes -> float64 values."""
    return _DEC[np.asarray(q, dtype=np.uint8)]


def encode(v) -> np.ndarray:
    """float32 -> e4m3fn codes, round-to-nearest-even, saturating at +-448.

    Every step is exact in float32 except the single rounding to a 3-bit
    mantissa, so this is a correctly rounded conversion: scale by a power of
    two into [8, 16) (normal) or [0, 8] (subnormal, unit 2^-9), round with
    rint (ties to even), rebuild the code.
    """
    v = np.asarray(v, dtype=_F32)
    a = np.abs(v).astype(np.float64)
    sign = np.where(np.signbit(v), 0x80, 0).astype(np.int64)
    out = np.zeros(v.shape, dtype=np.int64)
    nan = np.isnan(v)
    sat = (~nan) & (a >= E4M3_MAX)
    sub = (~nan) & (a < 2.0 ** -6)
    nor = (~nan) & (~sat) & (~sub)
    # subnormal: units of 2^-9; m == 8 is exactly the smallest normal (code 8)
    m_sub = np.rint(a[sub] * 2.0 ** 9).astype(np.int64)
    out[sub] = m_sub
    an = a[nor]
    e = np.floor(np.log2(an)).astype(np.int64)
    # guard log2 rounding at exact powers of two
    e = np.where(np.exp2(e.astype(np.float64)) > an, e - 1, e)
    e = np.where(np.exp2((e + 1).astype(np.float64)) <= an, e + 1, e)
    m = np.rint((an / np.exp2(e.astype(np.float64)) - 1.0) * 8.0).astype(np.int64)
    carry = m == 8
    e = np.where(carry, e + 1, e)
    m = np.where(carry, 0, m)
    code = ((e + 7) << 3) | m
    # 464 <= a < 480 cannot reach here (saturated above); a in [448, 464)
    # rounds to 448 either way
    out[nor] = code
    out[sat] = 0x7E
    out[nan] = 0x7F
    return (out | sign).astype(np.uint8)


def quantize_weight_blocks(w: np.ndarray, block: int = 128):
    """[R, C] float -> (q uint8 [R, C], scale_inv float32 [R/128, C/128]).

    scale_inv = amax(|block|) / 448 in float32; q = e4m3(w / scale_inv).
    This is the seeded-workload recipe ("per 128x128 block scale_inv =
    amax/448, q = e4m3fn(w/scale_inv), RNE, saturating").  An all-zero block
    gets scale_inv 1.0 and zero codes.
    """
    w = np.asarray(w, dtype=_F32)
    R, C = w.shape
    assert R % block == 0 and C % block == 0, (R, C)
    blocks = w.reshape(R // block, block, C // block, block)
    amax = np.abs(blocks).max(axis=(1, 3)).astype(_F32)
    scale = (amax / _F32(E4M3_MAX)).astype(_F32)
    scale = np.where(amax == 0, _F32(1.0), scale).astype(_F32)
    q = encode((blocks / scale[:, None, :, None]).astype(_F32))
    return q.reshape(R, C), scale


def dequantize_blocks(q: np.ndarray, scale_inv: np.ndarray, block: int = 128) -> np.ndarray:
    """Upstream dequantize_fp8_blocks restated (notes/13-non-ada-gpus.md:43-53):
    q [..., R, C] uint8, scale_inv [..., R/128, C/128] -> float64 [..., R, C]."""
    vals = decode(q)
    s = np.repeat(np.repeat(np.asarray(scale_inv, dtype=np.float64), block, axis=-2),
                  block, axis=-1)
    return vals * s


def quantize_activation(x: np.ndarray, group: int = 128):
    """Per row, per `group` columns: scale = amax/448 (float32), q = e4m3(x/scale).

    x [T, D] float32 -> (q uint8 [T, D], scale float32 [T, D/group]).
    Division is float32 round-to-nearest; a zero group has scale 0, codes 0.
    """
    x = np.asarray(x, dtype=_F32)
    T, D = x.shape
    assert D % group == 0
    g = x.reshape(T, D // group, group)
    amax = np.abs(g).max(axis=2).astype(_F32)
    scale = (amax / _F32(E4M3_MAX)).astype(_F32)
    safe = np.where(scale == 0, _F32(1.0), scale).astype(_F32)
    with np.errstate(invalid="ignore"):
        q = encode((g / safe[:, :, None]).astype(_F32))
    q = np.where((scale == 0)[:, :, None], np.uint8(0), q)
    return q.reshape(T, D), scale


def bf16_round(x) -> np.ndarray:
    """float -> nearest bfloat16 (RNE), returned as float32 values."""
    x = np.asarray(x, dtype=_F32)
    b = x.view(np.uint32).astype(np.uint64)
    lsb = (b >> 16) & 1
    r = ((b + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(_F32).copy()
    out[np.isnan(x)] = np.nan
    return out


def bf16_bits(x) -> np.ndarray:
    """float -> bfloat16 bit patterns (uint16), RNE."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b) -> np.ndarray:
    """uint16 bfloat16 bit patterns -> float32."""
    return (np.asarray(b, dtype=np.uint32) << 16).view(_F32)
