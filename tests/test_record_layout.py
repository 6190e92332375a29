"""The packed records' MFMA tile order (hostpool.to_tiles / from_tiles,
MOE_LAYOUT_TILES in include/moe_offload.h).

Checked on the CPU: every byte of a tiled matrix sits where the header's
formula puts it, (g*K/128 + b)*2048 + h*1024 + (16q + r)*16 + i for byte
(16g + r, 128b + 32q + 16h + i); the formula hands each lane of a wave the
32 bytes the row-major MFMA operand load gives it (lane 16q + r: row r,
reduction indices 32q..32q+31); from_tiles inverts to_tiles for torch and
numpy, batched; pack/unpack round-trip a record; tiled=False is plain
row-major; the loader writes the same records as pack in both orders.  The
GPU tests run the kernels on tiled records against the same experts in
row-major buffers, bit for bit."""
import numpy as np
import torch

import hostpool
from hostpool import RecordLayout, from_tiles, to_tiles


def _where(row, col, K):
    g, r = divmod(row, 16)
    b, c = divmod(col, 128)
    q, c = divmod(c, 32)
    h, i = divmod(c, 16)
    return (g * (K // 128) + b) * 2048 + h * 1024 + (16 * q + r) * 16 + i


def test_every_byte_where_the_formula_puts_it():
    R, K = 48, 384
    w = np.arange(R * K, dtype=np.int64).reshape(R, K)
    flat = to_tiles(w).reshape(-1)
    rows, cols = np.meshgrid(np.arange(R), np.arange(K), indexing="ij")
    pos = np.vectorize(lambda r, c: _where(r, c, K))(rows, cols)
    assert np.array_equal(flat[pos], w)
    assert np.array_equal(np.sort(pos.reshape(-1)), np.arange(R * K))   # a permutation


def test_lanes_get_the_row_major_operand_bytes():
    """Lane l = 16q + r of a wave loading row group g, K-block b reads
    [lo | hi] = tile + l*16 and tile + 1024 + l*16: the 32 bytes of row
    16g + r at columns 128b + 32q .. +32, as the row-major load does."""
    R, K = 32, 256
    w = np.random.default_rng(0).integers(0, 256, (R, K), dtype=np.uint8)
    flat = to_tiles(w).reshape(-1)
    for g in range(R // 16):
        for b in range(K // 128):
            tile = (g * (K // 128) + b) * 2048
            for lane in range(64):
                q, r = divmod(lane, 16)
                got = np.concatenate([flat[tile + lane * 16:][:16],
                                      flat[tile + 1024 + lane * 16:][:16]])
                assert np.array_equal(got, w[16 * g + r, 128 * b + 32 * q:][:32])


def test_inverse_torch_and_numpy_batched():
    g = torch.Generator().manual_seed(1)
    w = torch.randint(0, 256, (3, 64, 256), dtype=torch.uint8, generator=g)
    t = to_tiles(w)
    assert t.shape == w.shape and not torch.equal(t, w)
    assert torch.equal(from_tiles(t), w)
    assert np.array_equal(to_tiles(w.numpy()), t.numpy())
    assert np.array_equal(from_tiles(t.numpy()), w.numpy())
    # e4m3 views tile as bytes
    assert torch.equal(to_tiles(w.view(torch.float8_e4m3fn)).view(torch.uint8), t)


def test_pack_unpack_round_trip_and_row_order():
    H, I = 256, 128
    g = torch.Generator().manual_seed(2)
    w13 = torch.randint(0, 256, (2, 2 * I, H), dtype=torch.uint8, generator=g)
    w2 = torch.randint(0, 256, (2, H, I), dtype=torch.uint8, generator=g)
    s13 = torch.rand((2, 2 * I // 128, H // 128), generator=g)
    s2 = torch.rand((2, H // 128, I // 128), generator=g)
    e4 = torch.float8_e4m3fn
    for tiled in (True, False):
        lay = RecordLayout(H, I, tiled=tiled)
        assert lay.code == (hostpool.hipfetch.LAYOUT_TILES if tiled else hostpool.hipfetch.LAYOUT_ROWS)
        rec = lay.pack(w13.view(e4), s13, w2.view(e4), s2)
        for got, want in zip(lay.unpack(rec), (w13, s13, w2, s2)):
            assert torch.equal(got, want)
        for got, want in zip(lay.unpack(rec.numpy()), (w13, s13, w2, s2)):
            assert np.array_equal(got, want.numpy())
        raw13 = rec[:, :lay.off_w2].reshape(2, 2 * I, H)
        assert torch.equal(raw13, to_tiles(w13) if tiled else w13)
    assert hostpool.DRAMA3.tiled


def test_loader_records_in_both_orders(tmp_path):
    import loader
    from test_loader import _expert, _write_shards
    tensors = _write_shards(tmp_path, seed=5)
    index = loader.ShardIndex.from_dir(tmp_path)
    for tiled in (True, False):
        lay = RecordLayout(256, 128, tiled=tiled)
        dst = np.zeros((6, lay.record_bytes), np.uint8)
        loader.fill_records(index, 1, dst, lay, threads=2)
        for e in (0, 5):
            g, u, d = _expert(tensors, 1, e, "weight")
            gs, us, ds = _expert(tensors, 1, e, "weight_scale_inv")
            want = lay.pack(torch.cat([g, u])[None], torch.cat([gs, us])[None], d[None], ds[None])
            assert np.array_equal(dst[e], want[0].numpy())
