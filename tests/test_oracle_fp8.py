"""Pin the oracle's fp8/bf16 arithmetic against library routines and closed forms."""
import numpy as np
import pytest
import torch

from oracle import fp8


def test_decode_table_matches_torch_for_every_code():
    codes = torch.arange(256, dtype=torch.uint8)
    want = codes.view(torch.float8_e4m3fn).to(torch.float32).numpy().astype(np.float64)
    got = fp8.decode_table()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6


def _all_finite_values():
    t = fp8.decode_table()
    v = np.unique(t[~np.isnan(t)])
    return v


def test_encode_matches_torch_cast_including_ties():
    v = _all_finite_values()
    mids = (v[:-1] + v[1:]) / 2                     # exact ties
    rng = np.random.default_rng(0)
    rand = rng.uniform(-463.0, 463.0, 200_000)
    small = rng.uniform(-0.02, 0.02, 100_000)
    xs = np.concatenate([v, mids, np.nextafter(mids, 0), np.nextafter(mids, 1e9), rand, small])
    xs = xs[np.abs(xs) < 464].astype(np.float32)
    want = torch.from_numpy(xs).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = fp8.encode(xs)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (xs[bad[:5]], got[bad[:5]], want[bad[:5]])


def test_encode_saturates_and_keeps_nan():
    got = fp8.encode(np.array([448.0, 463.9, 464.0, 1e6, -1e6, np.inf, -np.inf, np.nan],
                              np.float32))
    assert list(got[:7]) == [0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0x7E, 0xFE]
    assert got[7] & 0x7F == 0x7F


def test_weight_block_quantisation_closed_form():
    """w = decode(q0) * s[block] with power-of-two scales and a 448 in every
    block must quantise back to exactly (q0, s); distinct scales per block on
    a non-square block grid catch a transposed block index."""
    rng = np.random.default_rng(1)
    R, C = 384, 256                                  # 3 x 2 blocks
    finite = np.flatnonzero(~np.isnan(fp8.decode_table()))
    q0 = rng.choice(finite, size=(R, C)).astype(np.uint8)
    for rb in range(3):
        for cb in range(2):
            q0[rb * 128, cb * 128] = 0x7E               # amax of every block is 448
    s = np.array([[2.0 ** -3, 2.0 ** -5], [2.0 ** -7, 2.0 ** 1], [2.0 ** -1, 2.0 ** -9]],
                 np.float32)
    w = (fp8.decode(q0) * np.repeat(np.repeat(s, 128, 0), 128, 1)).astype(np.float32)
    q, sc = fp8.quantize_weight_blocks(w)
    assert np.array_equal(sc, s)
    # +-0 both decode to 0; compare values
    assert np.array_equal(fp8.decode(q), fp8.decode(q0))
    back = fp8.dequantize_blocks(q, sc)
    assert np.array_equal(back, w.astype(np.float64))


def test_activation_quantisation_closed_form():
    x = np.zeros((2, 256), np.float32)
    x[0, :128] = np.linspace(-3.5, 3.5, 128)       # amax 3.5
    x[0, 128:] = 0.0                                # zero group
    x[1, :128] = 1.0
    x[1, 128:] = -2.0 ** -20
    q, s = fp8.quantize_activation(x)
    assert s[0, 0] == np.float32(3.5) / np.float32(448) and s[0, 1] == 0
    assert np.all(q[0, 128:] == 0)
    assert fp8.decode(q[0, 127]) == 448.0 and fp8.decode(q[0, 0]) == -448.0
    assert np.all(fp8.decode(q[1, :128]) == 448.0)
    assert np.all(fp8.decode(q[1, 128:]) == -448.0)


def test_torch_block_quantiser_matches_oracle():
    import synth
    g = torch.Generator().manual_seed(3)
    w = torch.randn((256, 384), generator=g) * 0.02
    w[0, 0] = 0.0
    qt, st = synth.quantize_blocks(w)
    qo, so = fp8.quantize_weight_blocks(w.numpy())
    assert np.array_equal(st.numpy(), so)
    assert np.array_equal(qt.numpy(), qo)


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(4)
    x = np.concatenate([rng.standard_normal(100_000) * 10 ** rng.uniform(-6, 6, 100_000),
                        [0.0, -0.0, 1.0, 65504.0, 3.0e38]]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(fp8.bf16_round(x), want)
    bits = fp8.bf16_bits(x)
    assert np.array_equal(fp8.bf16_from_bits(bits), want)
