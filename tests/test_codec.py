"""Coded records on the CPU: the library's encoder against the format's
independent restatement (oracle/codec.py) byte for byte, decode back to the
original records, code lengths against an exhaustive optimum, and the
decoder table against the canonical codes."""
import itertools

import numpy as np
import pytest
import torch

from oracle import codec as ocodec


def _records(seed, n, H=256, I=128, recipe="blockq"):
    import synth
    from hostpool import RecordLayout
    lay = RecordLayout(H, I)
    recs = []
    for e in range(n):
        a, b, c, d = synth.expert_tensors(seed, 0, e, H, I, recipe)
        recs.append(lay.pack(a[None], b[None], c[None], d[None])[0].numpy())
    return lay, np.stack(recs)


def test_code_lengths_are_optimal_length_limited_codes():
    import codec
    rng = np.random.default_rng(0)
    for trial in range(40):
        n = int(rng.integers(2, 7))
        L = int(rng.integers(max(2, int(np.ceil(np.log2(n)))), 5))
        hist = rng.integers(0, 1000, n) ** 2
        got = codec.code_lengths(hist, L)
        w = hist + 1
        assert sum(2.0 ** -int(l) for l in got) <= 1.0 + 1e-12
        assert got.max() <= L and got.min() >= 1
        best = min(sum(int(a) * b for a, b in zip(ls, w))
                   for ls in itertools.product(range(1, L + 1), repeat=n)
                   if sum(2.0 ** -l for l in ls) <= 1.0)
        assert sum(int(a) * b for a, b in zip(got, w)) == best, (hist, got)


def test_library_encoder_matches_the_format_and_decodes_back(lib):
    import codec
    lay, recs = _records(3, 2)
    fp8 = lay.off_s13
    hist = lib.codec_histogram(recs, fp8)
    assert int(hist.sum()) == 2 * fp8
    lengths = codec.code_lengths(hist)
    scratch = np.zeros(lib.codec_bound(lay.record_bytes, fp8) * 2, np.uint8)
    used, rec_off, blk_off = lib.codec_encode(recs, fp8, lengths, scratch, threads=2)
    assert used == rec_off[-1] and used % 256 == 0 and used < recs.nbytes
    for r in range(2):
        blob, offs = ocodec.encode_record(recs[r], fp8, lengths)
        mine = scratch[rec_off[r]:rec_off[r + 1]].tobytes()
        assert mine == blob, f"record {r}: library bytes differ from the format"
        assert list(blk_off[r]) == offs
        back = ocodec.decode_record(mine, offs, fp8, lay.record_bytes, lengths)
        assert np.array_equal(back, recs[r])


def test_every_byte_value_round_trips(lib):
    """All 256 e4m3 codes (NaNs and zeros too) through one block."""
    import codec
    x = np.tile(np.arange(256, dtype=np.uint8), 32)
    np.random.default_rng(1).shuffle(x)
    lengths = codec.code_lengths(np.bincount((x >> 3) & 15, minlength=16))
    blob = ocodec.encode_block(x, lengths)
    assert np.array_equal(ocodec.decode_block(blob, lengths), x)
    rec = np.concatenate([x, np.arange(256, dtype=np.uint8)])[None]     # 1 block + a 256-byte tail
    scratch = np.zeros(lib.codec_bound(rec.shape[1], 8192), np.uint8)
    used, rec_off, blk_off = lib.codec_encode(rec, 8192, lengths, scratch)
    assert scratch[:blk_off[0, 1]].tobytes() == blob


def test_decoder_table_matches_canonical_codes(lib):
    """Entry p: the two codes the stream bits p (least significant first)
    begin with, per the canonical codes of the oracle."""
    import codec
    lengths = codec.code_lengths([1, 1, 2, 3, 5, 8, 20, 60, 150, 300, 700, 1500, 3000, 4000,
                                  2500, 300])
    assert lengths.max() <= 6
    lut = lib.codec_table(lengths)
    by_code = {v: s for s, v in ocodec.canonical(lengths).items()}
    for p in range(4096):
        bits = [(p >> k) & 1 for k in range(12)]
        syms, i = [], 0
        for _ in range(2):
            c, ln = 0, 0
            while (c, ln) not in by_code:
                c, ln, i = (c << 1) | bits[i], ln + 1, i + 1
            syms.append(by_code[(c, ln)])
        assert lut[p] == syms[0] | syms[1] << 4 | i << 8, p


def test_bad_codes_are_refused(lib):
    lay, recs = _records(5, 1)
    scratch = np.zeros(lib.codec_bound(lay.record_bytes, lay.off_s13), np.uint8)
    import hipfetch
    with pytest.raises(hipfetch.NativeError, match="prefix code"):
        lib.codec_encode(recs, lay.off_s13, [1] * 16, scratch)            # Kraft sum 8
    with pytest.raises(hipfetch.NativeError, match="no code"):
        lib.codec_encode(recs, lay.off_s13, [0] * 8 + [3] * 8, scratch)   # exponents 0..7 uncoded
    with pytest.raises(hipfetch.NativeError, match="prefix code"):
        lib.codec_table([7] + [4] * 15)                                     # longer than 6


def test_synthetic_experts_code_to_about_84_percent(lib):
    import codec
    lay, recs = _records(0, 2, H=2048, I=512)
    fp8 = lay.off_s13
    lengths = codec.code_lengths(lib.codec_histogram(recs, fp8))
    scratch = np.zeros(lib.codec_bound(lay.record_bytes, fp8) * 2, np.uint8)
    used, _, _ = lib.codec_encode(recs, fp8, lengths, scratch)
    ratio = used / recs.nbytes
    print(f"coded / raw = {ratio:.4f}")
    assert 0.80 < ratio < 0.88
