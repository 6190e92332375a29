"""The kernels' e4m3 encoder (csrc/e4m3.hpp, built here for the host) against
the oracle's encoder and torch's float8_e4m3fn cast.

The header is compiled with g++ exactly as the kernels include it; every step
of the encoder is integer arithmetic or an exact float scaling followed by
one rintf, so host and device give the same codes."""
import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import fp8

ROOT = Path(__file__).resolve().parent


@pytest.fixture(scope="module")
def enc(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    so = tmp_path_factory.mktemp("e4m3") / "libe4m3host.so"
    subprocess.run([gxx, "-O2", "-std=c++20", "-shared", "-fPIC", "-o", str(so),
                    str(ROOT / "native" / "e4m3_host.cpp")], check=True)
    lib = ctypes.CDLL(str(so))
    lib.encode_many.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    lib.encode_range.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
    lib.quant_many.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    return lib


def _encode(lib, v):
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty(v.shape, np.uint8)
    lib.encode_many(v.ctypes.data, out.ctypes.data, v.size)
    return out


def test_every_tie_and_neighbour_matches_oracle(enc):
    """Every e4m3 value, every midpoint between neighbours and the floats one
    ulp either side of each, both signs."""
    vals = np.sort(fp8.decode(np.arange(0, 0x7f, dtype=np.uint8)).astype(np.float32))
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)
    pts = np.concatenate([vals, mids, np.nextafter(mids, np.float32(0)),
                          np.nextafter(mids, np.float32(np.inf)),
                          np.float32([447.99, 448, 455.9, 456, 464, 1e30, np.inf, 2.0 ** -10,
                                      2.0 ** -130, 0.0])])
    pts = np.concatenate([pts, -pts]).astype(np.float32)
    assert np.array_equal(_encode(enc, pts), fp8.encode(pts))
    nan = _encode(enc, np.float32([np.nan, -np.nan]))
    assert (nan & 0x7f).tolist() == [0x7f, 0x7f]


def test_exhaustive_in_range_matches_torch_cast(enc):
    """Every positive float in [2^-12, 448) (20 binades x 2^23 floats) against
    torch's float32 -> float8_e4m3fn cast, the reference's activation cast."""
    lo, hi = np.float32(2.0 ** -12).view(np.uint32), np.float32(448.0).view(np.uint32)
    step = 1 << 24
    for a in range(int(lo), int(hi), step):
        b = min(a + step, int(hi))
        out = np.empty(b - a, np.uint8)
        enc.encode_range(a, b, out.ctypes.data)
        v = torch.from_numpy(np.arange(a, b, dtype=np.uint32).view(np.float32))
        want = v.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        bad = np.flatnonzero(out != want)
        assert bad.size == 0, f"{bad.size} mismatches, first at bits {a + int(bad[0]):#x}"


def test_random_wide_range_and_quantiser_match_oracle(enc):
    rng = np.random.default_rng(5)
    v = (rng.standard_normal(1 << 20) * np.exp2(rng.uniform(-24, 12, 1 << 20))).astype(np.float32)
    assert np.array_equal(_encode(enc, v), fp8.encode(v))
    # quant_e4m3(v, s) = encode(v / s) with the float32 quotient, 0 for s == 0
    s = np.abs(rng.standard_normal(1 << 16)).astype(np.float32) / np.float32(448)
    s[::97] = 0
    x = rng.standard_normal(1 << 16).astype(np.float32)
    out = np.empty(x.shape, np.uint8)
    enc.quant_many(x.ctypes.data, s.ctypes.data, out.ctypes.data, x.size)
    with np.errstate(divide="ignore", invalid="ignore"):
        want = np.where(s == 0, 0, fp8.encode((x / s).astype(np.float32)))
    assert np.array_equal(out, want)
