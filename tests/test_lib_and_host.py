"""CPU-only checks: the C-ABI library loads and exports every declared entry
point, preconditions are rejected before anything is launched, and the host
logic of the hook surface behaves as the reference's does."""
import ctypes

import numpy as np
import pytest
import torch


def test_library_exports_every_declared_symbol(lib):
    import hipfetch
    declared = hipfetch.declared_symbols()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib.cdll, name), name
    assert set(declared) == set(hipfetch.SIGNATURES)


def test_phase_marks_build_is_separate(lib):
    """The decode GEMV's phase marks live only in libmoeoffload_marks.so (the
    bench's gemvphases probe), which exports the product's symbols too."""
    import subprocess
    import sys
    import hipfetch
    assert not hasattr(lib.cdll, "moe_phase_marks_read")
    marks = hipfetch.LIB_PATH.parent / "libmoeoffload_marks.so"
    if not marks.exists():
        pytest.skip("marks build not present")
    names = ["moe_phase_marks_read", "moe_phase_marks_clock_khz", *hipfetch.declared_symbols()]
    code = ("import ctypes, sys; l = ctypes.CDLL(sys.argv[1]); "
            "print(' '.join(n for n in sys.argv[2:] if not hasattr(l, n)))")
    out = subprocess.run([sys.executable, "-c", code, str(marks), *names],
                         stdout=subprocess.PIPE, text=True, timeout=120, check=True)
    assert out.stdout.strip() == ""


def test_library_shares_torchs_hip_runtime(lib):
    import hipfetch
    ours = lib.hip_runtime_path()
    assert ours.endswith(".so") or ".so." in ours
    theirs = hipfetch._torch_hip_runtime()
    if theirs:
        import os
        assert os.path.realpath(ours) == os.path.realpath(theirs)


def test_preconditions_are_rejected_without_launching(lib):
    c = lib.cdll
    pairs = (ctypes.c_byte * 64)()
    assert c.moe_fetch(ctypes.cast(pairs, ctypes.POINTER(__import__("hipfetch").FetchPair)), 5,
                       1, 1, 1, 8, 64, None) == -1
    assert b"npairs" in c.moe_last_error()
    p = ctypes.c_void_p()
    assert c.moe_host_alloc(ctypes.byref(p), 16, 7) == -1
    assert c.moe_slots_init(1, 256, 1, 1, 5000, 1, None) == -1
    assert b"cap" in c.moe_last_error()
    assert c.moe_fp8_moe_forward(1, 1, 0, 1, 2, 1, 8, 16, 1, 16, 1, 4, 2000, 512, 1, 16, 1 << 30,
                                 None) == -1
    assert b"hidden" in c.moe_last_error()
    bf16 = 3                                   # MOE_BF16 logits
    assert c.moe_router_topk(16, 16, None, bf16, 1, 2048, 256, 40, 1, 1, 0, 1, 2, None) == -1
    assert c.moe_router_topk(16, 16, None, 0, 1, 2048, 256, 8, 1, 1, 0, 1, 2, None) == -1
    assert b"logit_dtype" in c.moe_last_error()
    assert c.moe_route_resolve(16, 16, None, bf16, 2048, 256, 8, 1, 1, 1, 1, 1, 1, 9999, 1, 1, 1,
                               1, 1, None, None) == -1
    assert b"cap" in c.moe_last_error()
    # more ids than slots: one slot would go to two ids of the call
    assert c.moe_resolve_slots(1, 0, 9, 1, 256, 1, 1, 8, 1, 1, 1, 1, 1, None, None) == -1
    assert b"exceeds the cache capacity" in c.moe_last_error()
    assert c.moe_route_resolve(16, 16, None, bf16, 2048, 256, 8, 1, 1, 1, 1, 1, 1, 7, 1, 1, 1, 1,
                               1, None, None) == -1
    assert b"exceeds the cache capacity" in c.moe_last_error()
    # the three-launch decode layer: packed records of hidden % 512 == 0, top_k <= 16,
    # records that hold the layout, a workspace that holds the activations
    def rff(hidden=2048, top_k=8, cap=50, record_bytes=3146496, inter=512, pool=256, ws=1 << 20,
            wbytes=1 << 20):
        return c.moe_route_fetch_ffn(16, 16, None, bf16, hidden, 256, top_k, 1, 1, 1, 1, 1, 1,
                                     cap, 1, 1, 1, 1, 1, None, pool, 256, record_bytes, inter, 4,
                                     None, None, 256, ws, wbytes, None)
    for kw, msg in ((dict(hidden=1024 + 256), b"multiple of 512"),
                    (dict(top_k=17, cap=64), b"top_k"),
                    (dict(top_k=9, cap=8), b"exceeds the cache capacity"),
                    (dict(record_bytes=3146496 - 256), b"must hold"),
                    (dict(pool=264), b"256-byte aligned"),
                    (dict(wbytes=8 * 512 * 4 - 4), b"workspace")):
        assert rff(**kw) == -1, msg
        assert msg in c.moe_last_error(), (msg, c.moe_last_error())
    # its 0 %-hit form: the same checks, no table (a NULL one is no refusal)
    def rffu(hidden=2048, top_k=8, cap=8, record_bytes=3146496, inter=512, pool=256,
             ws=1 << 20, wbytes=1 << 20, ids=1):
        return c.moe_route_fetch_ffn_uncached(16, 16, None, bf16, hidden, 256, top_k, 1, ids, 1,
                                              cap, 1, 1, 1, 1, None, pool, 256, record_bytes,
                                              inter, 4, None, None, 256, ws, wbytes, None)
    for kw, msg in ((dict(hidden=1024 + 256), b"multiple of 512"),
                    (dict(top_k=17, cap=64), b"top_k"),
                    (dict(top_k=9, cap=8), b"exceeds the cache capacity"),
                    (dict(record_bytes=3146496 - 256), b"must hold"),
                    (dict(pool=264), b"256-byte aligned"),
                    (dict(wbytes=8 * 512 * 4 - 4), b"workspace"),
                    (dict(ids=None), b"NULL pointer")):
        assert rffu(**kw) == -1, msg
        assert msg in c.moe_last_error(), (msg, c.moe_last_error())
        assert c.moe_last_error().startswith(b"moe_route_fetch_ffn_uncached:")
    # the coded route + fetch: the route's limits and the coded fetch's record shape
    def rfc(top_k=8, cap=50, n_experts=256, record_bytes=3146496, fp8_bytes=3145728, pool=256,
            slot_bytes=3146496, workgroups=32):
        return c.moe_route_fetch_coded(16, 16, None, bf16, 2048, n_experts, top_k, 1, 1, 1, 1,
                                       1, 1, cap, 1, 1, 1, 1, 1, None, pool, 1, 1, record_bytes,
                                       fp8_bytes, 1, 256, slot_bytes, workgroups, None)
    for kw, msg in ((dict(top_k=33, cap=64), b"top_k"),
                    (dict(n_experts=1025), b"n_experts <= 1024"),
                    (dict(cap=1025), b"cap <= 1024"),
                    (dict(top_k=9, cap=8), b"exceeds the cache capacity"),
                    (dict(fp8_bytes=3145728 - 16), b"multiple of 8192"),
                    (dict(record_bytes=3145728 + 8), b"multiple of 8192"),
                    (dict(slot_bytes=3146496 - 16), b"at least one record"),
                    (dict(pool=272), b"256-byte"),
                    (dict(workgroups=0), b"workgroups")):
        assert rfc(**kw) == -1, msg
        assert msg in c.moe_last_error(), (msg, c.moe_last_error())
    # the router inside the GEMV's gate/up launch: 1..16 tokens, top_k <= 16,
    # n_experts <= 1024, and the expert call's own checks, all before a launch
    def rff_router(tokens=1, top_k=8, n_experts=256, hidden=2048, ws=1 << 20):
        return c.moe_router_fp8_moe_forward(16, 16, None, bf16, tokens, hidden, n_experts, top_k,
                                            1, 1, 1, 16, 1, 16, 1, 512, None, None, 1, 256, ws,
                                            None)
    for kw, msg in ((dict(tokens=0), b"tokens"), (dict(tokens=17), b"tokens"),
                    (dict(top_k=17), b"top_k"), (dict(n_experts=1025), b"n_experts"),
                    (dict(hidden=2000), b"hidden"), (dict(ws=16), b"workspace")):
        assert rff_router(**kw) == -1, msg
        assert msg in c.moe_last_error(), (msg, c.moe_last_error())
    # the stub product: 1..128 tokens; beyond 4, K % 64, N % 16 and no addend
    for args, msg in (((16, None, 16, 129, 64, 16, 16, 0, None), b"tokens"),
                      ((16, None, 16, 5, 72, 16, 16, 0, None), b"multiple of 64"),
                      ((16, None, 16, 5, 64, 8, 16, 0, None), b"multiple of 64"),
                      ((16, 16, 16, 5, 64, 16, 16, 0, None), b"x_add NULL"),
                      ((16, None, 16, 2, 64, 16, 16, 3, None), b"rows_per_wave")):
        assert c.moe_linear_bf16(*args) == -1, msg
        assert msg in c.moe_last_error(), (msg, c.moe_last_error())
    # tile-order pairs: K a multiple of 128, whole 16-row groups, 16-byte aligned
    FetchPair = __import__("hipfetch").FetchPair
    for src, dst, nbytes, tile_k, msg in ((0x1000, 0x2000, 16 * 256, 192, b"multiple of 128"),
                                          (0x1000, 0x2000, 8 * 256, 256, b"16 rows"),
                                          (0x1000, 0x2004, 16 * 256, 256, b"16-byte aligned"),
                                          (0x1000, 0x2000, 4096, -128, b"tile_k -128")):
        pair = FetchPair(src, dst, nbytes, tile_k)
        assert c.moe_fetch(ctypes.byref(pair), 1, 1, 1, 1, 8, 3, None) == -1, msg
        assert msg in c.moe_last_error(), c.moe_last_error()


def test_fetch_ffn_refuses_pairs_that_miss_the_cache_buffers(lib):
    """moe_fetch_ffn's down launch reads w2/s2 from the cache buffers it is
    given: pairs that fill other buffers, or strides that disagree with
    them, are refused before any launch (every case below fails a check
    ahead of the launch; none is ever well formed)."""
    import ctypes as C
    import hipfetch
    c = lib.cdll
    H, I = 2048, 512
    W13, W2, S13, S2 = 0x100000, 0x200000, 0x300000, 0x400000
    good = [(0x10000, W13, 2 * I * H, H), (0x20000, W2, H * I, I), (0x30000, S13, 512, 0),
            (0x40000, S2, 256, 0)]
    good_es = (2 * I * H, 128, H * I, 64)

    def call(pairs, es):
        arr = (hipfetch.FetchPair * 4)(*[hipfetch.FetchPair(*p) for p in pairs])
        st = hipfetch.ExpertStrides(*es, hipfetch.LAYOUT_TILES)
        one = C.c_void_p(256)
        return c.moe_fetch_ffn(arr, 4, one, one, one, 8, 3, one, one, one, hipfetch.MOE_F32, 8,
                               W13, S13, W2, S2, 16, H, I, C.byref(st), None, one, one, 1 << 20,
                               None)

    def with_pair(i, **kw):
        p = list(good[i])
        for k, v in kw.items():
            p[("src", "dst", "bytes", "tile_k").index(k)] = v
        return good[:i] + [tuple(p)] + good[i + 1:]

    cases = ((with_pair(1, dst=W2 + 256), good_es, b"w2 and s2"),
             (with_pair(3, dst=S13), good_es, b"w2 and s2"),
             (with_pair(3, bytes=512), good_es, b"pair 3 must be s2"),
             (with_pair(3, tile_k=128), good_es, b"pair 3 must be s2"),
             (good, (2 * I * H, 128, H * I + 256, 64), b"w2 and s2"),
             (good, (2 * I * H, 128, H * I, 128), b"w2 and s2"),
             (with_pair(0, dst=W2), good_es, b"w13 and s13"))
    for pairs, es, msg in cases:
        assert call(pairs, es) == -1, msg
        assert msg in c.moe_last_error(), (msg, c.moe_last_error())


def test_resolve_fetch_ffn_refuses_bad_tables(lib):
    """moe_resolve_fetch_ffn checks the ids dtype, the table's sizes and
    that the staging is not the table itself before any launch (each case
    below fails a check ahead of the launch)."""
    import ctypes as C
    import hipfetch
    c = lib.cdll
    H, I = 2048, 512
    W13, W2, S13, S2 = 0x100000, 0x200000, 0x300000, 0x400000
    pairs = (hipfetch.FetchPair * 4)(*[hipfetch.FetchPair(*p) for p in (
        (0x10000, W13, 2 * I * H, H), (0x20000, W2, H * I, I), (0x30000, S13, 512, 0),
        (0x40000, S2, 256, 0))])
    es = hipfetch.ExpertStrides(2 * I * H, 128, H * I, 64, hipfetch.LAYOUT_TILES)
    one = C.c_void_p(256)

    def call(ids_dtype=hipfetch.MOE_I32, top_k=8, E=256, cap=16, alias=False):
        t = hipfetch.SlotTable(0x1000, 0x2000, 0x3000, 0x4000, E, cap,
                               0x1000 if alias else 0x5000, 0x6000, 0x7000, 0x8000)
        return c.moe_resolve_fetch_ffn(one, ids_dtype, top_k, C.byref(t), one, one, one, one, None,
                                       pairs, 4, 3, one, one, hipfetch.MOE_F32, W13, S13, W2, S2,
                                       H, I, C.byref(es), None, one, one, 1 << 20, None)
    for kw, msg in ((dict(ids_dtype=hipfetch.MOE_F32), b"ids_dtype"),
                    (dict(E=2000), b"n_experts"),
                    (dict(cap=2000), b"cap"),
                    (dict(top_k=12, cap=10), b"exceeds the cache capacity"),
                    (dict(alias=True), b"staging"),
                    (dict(top_k=17, cap=20), b"top_k")):
        assert call(**kw) == -1, msg
        assert msg in c.moe_last_error(), (msg, c.moe_last_error())


def test_shared_and_block_preconditions_are_rejected_without_launching(lib):
    import ctypes as C
    import hipfetch
    c = lib.cdll
    one = C.c_void_p(16)                   # never dereferenced: every call fails a check first
    assert c.moe_shared_gate_up(one, one, one, one, 1, 2048, 500, one, one, None) == -1
    assert b"multiples of 128" in c.moe_last_error()
    assert c.moe_shared_gate_up(None, one, one, one, 1, 2048, 512, one, one, None) == -1
    assert b"NULL" in c.moe_last_error()
    assert c.moe_shared_gate_up(C.c_void_p(8), one, one, one, 1, 2048, 512, one, one, None) == -1
    assert b"aligned" in c.moe_last_error()
    assert c.moe_shared_gate_up(None, None, None, None, 0, 2048, 512, None, None, None) == 0
    assert c.moe_shared_down(one, one, one, 1, 2000, 512, None, None, one, None) == -1
    assert b"multiples of 128" in c.moe_last_error()
    assert c.moe_shared_down(None, None, None, 0, 2048, 512, None, None, None, None) == 0
    assert c.moe_e4m3_check(0, 16, None, None) == -1
    assert c.moe_e4m3_check(0, 0, one, None) == -1
    assert c.moe_e4m3_check(0xffffff00, 512, one, None) == -1
    assert c.moe_all_finite(one, 7, 4, one, None) == -1
    assert b"dtype" in c.moe_last_error()
    assert c.moe_all_finite(C.c_void_p(4), hipfetch.MOE_F32, 4, one, None) == -1
    assert b"aligned" in c.moe_last_error()
    # the block call: shared expert missing, misaligned, workspace too small
    es = hipfetch.ExpertStrides(2 * 512 * 2048, 8 * 16, 2048 * 512, 16 * 4)
    args = lambda sh, ws_bytes: (one, one, hipfetch.MOE_I32, one, hipfetch.MOE_F32, 1, 8, one, one,
                                 one, one, 16, 2048, 512, C.byref(es), sh, None, one, one,
                                 ws_bytes, 0, None)
    assert c.moe_fp8_moe_block_forward(*args(None, 1 << 30)) == -1
    assert b"shared expert" in c.moe_last_error()
    bad = hipfetch.SharedExpert(one, one, one, C.c_void_p(8), 512)
    assert c.moe_fp8_moe_block_forward(*args(C.byref(bad), 1 << 30)) == -1
    assert b"aligned" in c.moe_last_error()
    ok = hipfetch.SharedExpert(one, one, one, one, 512)
    need = c.moe_fp8_moe_block_workspace(1, 8, 16, 2048, 512, 512)
    assert need > c.moe_fp8_moe_workspace(1, 8, 16, 2048, 512)
    assert c.moe_fp8_moe_block_forward(*args(C.byref(ok), need - 1)) == -1
    assert b"workspace" in c.moe_last_error()
    odd = hipfetch.SharedExpert(one, one, one, one, 200)
    assert c.moe_fp8_moe_block_forward(*args(C.byref(odd), 1 << 30)) == -1
    assert b"shared inter" in c.moe_last_error()


def test_forward_modes(lib):
    """Modes 0-3 pass the preconditions (an empty call touches nothing);
    any other mode is refused before anything is enqueued."""
    import hipfetch
    c = lib.cdll
    for mode in range(4):
        assert c.moe_fp8_moe_forward_ex(None, None, hipfetch.MOE_I32, None, hipfetch.MOE_F32, 0, 8,
                                        None, None, None, None, 256, 2048, 512, None, None, None,
                                        None, 0, mode, None) == 0, mode
    for mode in (-1, 4):
        assert c.moe_fp8_moe_forward_ex(None, None, hipfetch.MOE_I32, None, hipfetch.MOE_F32, 0, 8,
                                        None, None, None, None, 256, 2048, 512, None, None, None,
                                        None, 0, mode, None) == -1
        assert b"mode must be 0, 1, 2 or 3" in c.moe_last_error()


def test_noalloc_forward_refuses_calls_beyond_its_scratch(lib):
    import ctypes as C
    import hipfetch
    c = lib.cdll
    one = C.c_void_p(16)                   # never dereferenced: the size check fails first
    es = hipfetch.ExpertStrides(2 * 512 * 2048, 8 * 16, 2048 * 512, 16 * 4)
    cap = 16 << 20
    # 512 tokens of top-8 (the prefill call) need about 35 MiB of workspace
    assert c.moe_fp8_moe_workspace(512, 8, 256, 2048, 512) > cap
    assert c.moe_fp8_moe_forward_noalloc(one, one, hipfetch.MOE_I32, one, hipfetch.MOE_F32, 512, 8,
                                         one, one, one, one, 256, 2048, 512, C.byref(es), None,
                                         one, 0, None) == -1
    assert b"more than the 16777216" in c.moe_last_error()
    # other preconditions are those of moe_fp8_moe_forward_ex
    assert c.moe_fp8_moe_forward_noalloc(one, one, hipfetch.MOE_I32, one, hipfetch.MOE_F32, 1, 8,
                                         one, one, one, one, 256, 2000, 512, None, None, one, 0,
                                         None) == -1
    assert b"hidden" in c.moe_last_error()
    # an empty call does nothing and needs no scratch
    assert c.moe_fp8_moe_forward_noalloc(None, None, hipfetch.MOE_I32, None, hipfetch.MOE_F32, 0,
                                         8, None, None, None, None, 256, 2048, 512, None, None,
                                         None, 0, None) == 0
    # decode and batches up to ~160 tokens fit
    assert c.moe_fp8_moe_workspace(128, 8, 256, 2048, 512) <= cap


def test_workspace_size_formula(lib):
    def al(v):
        return (v + 255) // 256 * 256

    def grouped(T, K, E, H, I):
        P = T * K
        max_tiles = (P + 31) // 32 + E              # 32-token work tiles, one list entry each
        return (al(4 * E) + al(4 * (E + 1)) + 2 * al(4 * P) + al(8 * max_tiles) + al(4)
                + al(T * H) + al(4 * T * H // 128) + al(4 * P * 2 * I)
                + al(P * I) + al(4 * P * I // 128) + al(4 * P * H))

    for T in (1, 2, 5, 512):
        gemv = al(T * 8 * 1024 * 4)
        assert lib.fp8_moe_workspace(T, 8, 256, 2048, 512) == max(gemv, grouped(T, 8, 256, 2048, 512))


def test_loader_contract_missing_library(tmp_path, monkeypatch):
    import hipfetch
    monkeypatch.setattr(hipfetch, "LIB_PATH", tmp_path / "nope.so")
    hipfetch.reset()
    try:
        assert hipfetch.load() is None
        assert "missing" in hipfetch.last_error()
        with pytest.raises(RuntimeError, match="unavailable"):
            hipfetch.require()
    finally:
        monkeypatch.undo()
        hipfetch.reset()
        assert hipfetch.load() is not None


def test_fetch_backend_knob(lib):
    import devcache

    class Fake:
        _dc_cap = 4
        _dc_out = torch.zeros(8, dtype=torch.int32)

    devcache.FETCH_BACKEND = "bogus"
    try:
        with pytest.raises(ValueError, match="FETCH_BACKEND"):
            devcache.dev_resolve_and_fetch(Fake(), torch.zeros((1, 8), dtype=torch.long))
    finally:
        devcache.FETCH_BACKEND = "hip"
    # more ids than slots is refused before anything is enqueued
    with pytest.raises(ValueError, match="capacity"):
        devcache.dev_resolve_and_fetch(Fake(), torch.zeros((1, 8), dtype=torch.long))


def test_capacity_sizing_arithmetic():
    import offload
    GiB = 2 ** 30
    # (free - (2 + 1.5) GiB) // (40 * 3,146,496)  (bin/offload.py:641-646)
    assert offload.capacity_for_free_vram(None, 40, 256, free_bytes=20 * GiB) == \
        int((20 - 3.5) * GiB // (40 * 3_146_496))
    assert offload.capacity_for_free_vram(None, 40, 256, free_bytes=3 * GiB) == 0
    assert offload.capacity_for_free_vram(None, 40, 256, free_bytes=280 * GiB) == 256
    assert offload.capacity_for_free_vram(None, 40, 256, free_bytes=280 * GiB,
                                          cap_per_layer=96) == 96
    # the experts' own size when they are not Drama-3's
    assert offload.capacity_for_free_vram(None, 4, 32, free_bytes=4 * GiB,
                                          expert_bytes=1 << 20) == 32
    assert offload.capacity_for_free_vram(None, 4, 256, free_bytes=4 * GiB,
                                          expert_bytes=1 << 20) == \
        int((4 - 3.5) * GiB // (4 << 20))


def test_fp8_moe_forward_has_no_cpu_path(lib):
    from fp8_moe import fp8_moe_forward
    x = torch.zeros((1, 256), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        fp8_moe_forward(x, torch.zeros((1, 1), dtype=torch.long), torch.ones((1, 1)),
                        torch.zeros((1, 256, 256), dtype=torch.float8_e4m3fn),
                        torch.ones((1, 2, 2)),
                        torch.zeros((1, 256, 128), dtype=torch.float8_e4m3fn),
                        torch.ones((1, 2, 1)))


def test_wrappers_refuse_host_tensors(lib):
    # a CPU tensor's address handed to a kernel would fault the device
    i32 = lambda n: torch.zeros(n, dtype=torch.int32)
    with pytest.raises(ValueError, match="on the GPU"):
        lib.resolve_slots(i32(8), i32(256), i32(64), torch.zeros(64, dtype=torch.int64),
                          torch.zeros(1, dtype=torch.int64), i32(8), i32(8), i32(8), i32(1))
    with pytest.raises(ValueError, match="on the GPU"):
        lib.fetch([(16, 16, 256)], i32(8), i32(8), i32(1), max_jobs=8, blocks_per_job=2)
    x = torch.zeros((1, 2048), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="on the GPU"):
        lib.router_topk(x, torch.zeros((256, 2048), dtype=torch.bfloat16), None, 8,
                        torch.zeros((1, 256)), torch.zeros((1, 8), dtype=torch.int64),
                        torch.zeros((1, 8)))


def test_wrappers_check_buffer_sizes_and_dtypes(lib, monkeypatch):
    # The kernels index the table, list and output buffers by the sizes
    # passed beside them: a short, strided or differently typed buffer is
    # refused before anything reaches the library, and a well-formed call
    # gets through (the stand-in library below raises when called).
    class NoCall:
        def __getattr__(self, name):
            def f(*a):
                raise AssertionError(f"{name} reached")
            return f
    monkeypatch.setattr(lib, "_on_gpu", lambda *a: None)
    monkeypatch.setattr(lib, "cdll", NoCall())
    monkeypatch.setattr(lib, "stream", lambda: 0)
    i32 = lambda *n: torch.zeros(n, dtype=torch.int32)
    i64 = lambda *n: torch.zeros(n, dtype=torch.int64)
    E, C, K, H = 256, 64, 8, 2048

    def resolve(**over):
        a = dict(ids=i32(K), slot_of=i32(E), slot_expert=i32(C), stamp=i64(C), step=i64(1),
                 out_slot=i32(K), fetch_slot=i32(K), fetch_expert=i32(K), nmiss=i32(1),
                 stats=i64(2))
        a.update(over)
        lib.resolve_slots(**a)
    with pytest.raises(AssertionError, match="moe_resolve_slots reached"):
        resolve()
    for over, msg in ((dict(stamp=i32(C)), "stamp must be int64"),
                      (dict(stamp=i64(C - 1)), "stamp holds 63 elements, needs 64"),
                      (dict(out_slot=i32(K - 1)), "out_slot holds 7"),
                      (dict(fetch_expert=i64(K)), "fetch_expert must be int32"),
                      (dict(nmiss=i32(0)), "nmiss holds 0"),
                      (dict(stats=i64(1)), "stats holds 1"),
                      (dict(ids=torch.zeros(K)), "ids must be int32 or int64"),
                      (dict(slot_of=i32(2 * E)[::2]), "slot_of must be contiguous")):
        with pytest.raises(ValueError, match=msg):
            resolve(**over)

    with pytest.raises(ValueError, match="fetch_slot holds 4 elements, needs 8"):
        lib.fetch([(16, 16, 256)], i32(8), i32(4), i32(1), max_jobs=8, blocks_per_job=3)
    with pytest.raises(ValueError, match="moe_slots_init: stamp holds"):
        lib.slots_init(i32(E), i32(C), i64(C - 1), i64(1))

    x, w = torch.zeros((1, H), dtype=torch.bfloat16), torch.zeros((E, H), dtype=torch.bfloat16)

    def topk(**over):
        a = dict(x=x, w=w, bias=None, top_k=K, logits=torch.zeros(1, E), ids=i32(1, K),
                 weights=torch.zeros(1, K))
        a.update(over)
        lib.router_topk(**a)
    with pytest.raises(AssertionError, match="moe_router_topk reached"):
        topk()
    for over, msg in ((dict(logits=torch.zeros(E - 1)), "logits holds 255"),
                      (dict(x=x.float()), "x must be bfloat16"),
                      (dict(w=torch.zeros((E, H + 8), dtype=torch.bfloat16)), "share H"),
                      (dict(bias=torch.zeros(E, dtype=torch.bfloat16)), "bias must be float32"),
                      (dict(ids=i32(1, K - 1)), "ids holds 7"),
                      (dict(weights=torch.zeros(1, K, dtype=torch.float64)), "weights must be")):
        with pytest.raises(ValueError, match=msg):
            topk(**over)

    def route_fetch(**over):
        a = dict(x=x, w=w, bias=None, top_k=K, logits=torch.zeros(E), ids=i32(K),
                 weights=torch.zeros(K), slot_of=i32(2, E), slot_expert=i32(2, C),
                 stamp=i64(2, C), step=i64(1), out_slot=i32(K), fetch_slot=i32(K),
                 fetch_expert=i32(K), nmiss=i32(1), pairs=[(16, 16, 4096)], blocks_per_job=3)
        a.update(over)
        lib.route_fetch(**a)
    with pytest.raises(AssertionError, match="moe_route_fetch reached"):
        route_fetch()
    for over, msg in ((dict(ids=i64(K)), "ids must be int32"),
                      (dict(stamp=i32(2, C)), "stamp must be int64"),
                      (dict(fetch_slot=i32(K - 2)), "fetch_slot holds 6"),
                      (dict(stats=i32(2)), "stats must be int64")):
        with pytest.raises(ValueError, match=msg):
            route_fetch(**over)

    def route_fetch_coded(**over):
        a = dict(x=x, w=w, bias=None, top_k=K, logits=torch.zeros(E), ids=i32(K),
                 weights=torch.zeros(K), slot_of=i32(2, E), slot_expert=i32(2, C),
                 stamp=i64(2, C), step=i64(1), out_slot=i32(K), fetch_slot=i32(K),
                 fetch_expert=i32(K), nmiss=i32(1), pool_dev_ptr=256, rec_off=i64(E + 1),
                 blk_off=torch.zeros(E * 385, dtype=torch.uint32), record_bytes=3146496,
                 fp8_bytes=3145728, lut=torch.zeros(4096, dtype=torch.int16),
                 cache=torch.zeros((C, 3146496), dtype=torch.uint8, device="meta"))
        a.update(over)
        lib.route_fetch_coded(**a)
    with pytest.raises(AssertionError, match="moe_route_fetch_coded reached"):
        route_fetch_coded()
    for over, msg in ((dict(rec_off=i64(E)), "rec_off holds 256 elements, needs 257"),
                      (dict(blk_off=i32(E * 385 - 1)), "blk_off holds"),
                      (dict(lut=i32(4096)), "lut must be"),
                      (dict(slot_of=i32(2, E + 1)), "does not match"),
                      (dict(cache=torch.zeros((C - 1, 3146496), dtype=torch.uint8,
                                              device="meta")), "cache has 63 slots"),
                      (dict(cache=torch.zeros((C, 3146480), dtype=torch.uint8, device="meta")),
                       "record_bytes")):
        with pytest.raises(ValueError, match=msg):
            route_fetch_coded(**over)

    def route_fetch_ffn_uncached(**over):
        a = dict(x=x, w=w, bias=None, top_k=K, logits=torch.zeros(E), ids=i32(K),
                 weights=torch.zeros(K), out_slot=i32(K), fetch_slot=i32(K),
                 fetch_expert=i32(K), nmiss=i32(1), pool_dev_ptr=256,
                 cache=torch.zeros((K, 3146496), dtype=torch.uint8, device="meta"), inter=512,
                 blocks_per_job=4, out=torch.zeros((1, H), dtype=torch.bfloat16),
                 workspace=torch.zeros(1 << 16, dtype=torch.uint8))
        a.update(over)
        lib.route_fetch_ffn_uncached(**a)
    with pytest.raises(AssertionError, match="moe_route_fetch_ffn_uncached reached"):
        route_fetch_ffn_uncached()
    for over, msg in ((dict(ids=i64(K)), "ids must be int32"),
                      (dict(out_slot=i32(K - 1)), "out_slot holds 7"),
                      (dict(nmiss=i32(0)), "nmiss holds 0"),
                      (dict(stats=i32(2)), "stats must be int64"),
                      (dict(out=torch.zeros((1, H))), "out must be bfloat16"),
                      (dict(cache=torch.zeros((K, 3146496), dtype=torch.int8, device="meta")),
                       "cache must be contiguous uint8"),
                      (dict(shared=(torch.zeros((256, H), dtype=torch.bfloat16),) * 4),
                       "shared expert weights do not match")):
        with pytest.raises(ValueError, match=msg):
            route_fetch_ffn_uncached(**over)

    with pytest.raises(ValueError, match="offsets holds 256 elements, needs 257"):
        lib.permute(i32(4, K), E, i32(E), i32(E), i32(4 * K), i32(4 * K))
    with pytest.raises(ValueError, match="out must be bfloat16"):
        lib.unpermute(torch.zeros(4 * K, H), i32(4 * K), torch.zeros(4, K), torch.zeros(4, H))
    with pytest.raises(ValueError, match="uniq holds"):
        lib.unique_inverse(i32(4, K), E, i32(E), i32(1), i32(E - 1), i32(E), i32(4 * K))


def test_moe_experts_surface():
    import moe
    m = moe.MoEExperts(4, 256, 128)
    assert [n for n, _ in m.named_parameters()] == []          # buffers, not Parameters
    assert sorted(n for n, _ in m.named_buffers()) == ["w13_scale_inv", "w13_weight",
                                                       "w2_scale_inv", "w2_weight"]
    assert m.w13_weight.shape == (4, 256, 256) and m.w2_scale_inv.shape == (4, 2, 1)
    w = torch.arange(4 * 256 * 256, dtype=torch.int64).remainder(251).to(torch.uint8)
    m.w13_weight.view(torch.uint8).copy_(w.view(4, 256, 256))
    sel = moe.select_fp8(m.w13_weight, torch.tensor([2, 0]))
    assert torch.equal(sel.view(torch.uint8), m.w13_weight.view(torch.uint8)[[2, 0]])
    with pytest.raises(RuntimeError, match="host memory"):
        m(torch.zeros((1, 256), dtype=torch.bfloat16), torch.zeros((1, 1), dtype=torch.long),
          torch.ones((1, 1)))


def test_zipf_generators_are_seeded_and_distinct():
    import synth
    a = synth.zipf_miss_list(np.random.default_rng(1), 64)
    b = synth.zipf_miss_list(np.random.default_rng(1), 64)
    assert np.array_equal(a, b) and len(set(a.tolist())) == 64
    bias = synth.decode_route_bias(np.random.default_rng(0), 60, 2, 256, 1.1, 50)
    assert bias.shape == (60, 2, 256) and bias.dtype == np.float32


def test_install_offload_hooks_the_given_expert_class():
    """install_offload patches the class the model's experts are built from
    (upstream's MoEExperts in the reference's model) and keeps its resident
    forward as _stock_forward, idempotently (bin/offload.py:702-704)."""
    import moe
    import offload

    class Upstream(moe.MoEExperts):     # stands in for fish-speech's class
        def forward(self, x, topk_ids, topk_weights):
            return x

    orig = Upstream.forward
    offload.install_offload(Upstream)
    offload.install_offload(Upstream)
    assert Upstream.forward is offload.offloaded_forward
    assert Upstream._stock_forward is orig
    assert moe.MoEExperts.forward is not offload.offloaded_forward
