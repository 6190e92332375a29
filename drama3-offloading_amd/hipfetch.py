"""Load libmoeoffload.so, the HIP (gfx950) kernels of the expert-offload path.

Counterpart of bin/cppfetch.py: `load()` returns the bound library or None,
and never raises; `last_error()` says why it is None.  Unlike the reference,
nothing falls back to another backend when the library is missing: the
callers in devcache/offload/fp8_moe raise through `require()`, so a GPU run
without the native code fails loudly instead of silently running something
else.

The library is built in-tree by `python drama3-offloading_amd/build.py` (no
JIT, no per-user cache).  torch is imported before the library is opened so
that the library's libamdhip64.so.7 dependency resolves to the runtime torch
already loaded; `load()` verifies that, because a second HIP runtime in the
process would not understand torch's streams or allocations.
"""
from __future__ import annotations

import ctypes as C
import os
import weakref
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("MOE_OFFLOAD_LIB", HERE / "libmoeoffload.so"))

MOE_I32, MOE_I64, MOE_F32, MOE_BF16 = 0, 1, 2, 3

_lib = None
_err: str | None = None


def _free_host_buffer(lib, ptr: int, nbytes: int, hooks) -> None:
    """Finaliser of Lib.host_buffer's memory: its last view is gone."""
    for hook in hooks:
        try:
            hook(ptr, ptr + nbytes)
        except Exception:                                     # noqa: BLE001
            pass
    lib.host_free(ptr)


# byte order of the e4m3 expert matrices (moe_expert_strides.layout)
LAYOUT_ROWS = 0    # row-major, the checkpoint's nn.Linear layout
LAYOUT_TILES = 1   # MFMA tile order, the packed host records' layout


class ExpertStrides(C.Structure):
    """moe_expert_strides (include/moe_offload.h)."""
    _fields_ = [("w13", C.c_int64), ("s13", C.c_int64), ("w2", C.c_int64), ("s2", C.c_int64),
                ("layout", C.c_int64)]


def _expert_strides(w13, s13, w2, s2, layout: int) -> ExpertStrides:
    """Expert-axis strides of the four weight buffers (every other dimension
    contiguous) and their byte order."""
    for t in (w13, s13, w2, s2):
        if not t[0].is_contiguous():
            raise ValueError("expert weights must be contiguous within an expert")
    if layout not in (LAYOUT_ROWS, LAYOUT_TILES):
        raise ValueError(f"layout must be LAYOUT_ROWS or LAYOUT_TILES, got {layout!r}")
    return ExpertStrides(w13.stride(0), s13.stride(0), w2.stride(0), s2.stride(0), layout)


class SharedExpert(C.Structure):
    """moe_shared_expert (include/moe_offload.h)."""
    _fields_ = [("w_gate", C.c_void_p), ("w_up", C.c_void_p), ("w_down", C.c_void_p),
                ("w_sgate", C.c_void_p), ("inter", C.c_int32)]


class FetchPair(C.Structure):
    """moe_fetch_pair (include/moe_offload.h)."""
    _fields_ = [("src", C.c_void_p), ("dst", C.c_void_p), ("bytes", C.c_int64),
                ("tile_k", C.c_int64)]


class SlotTable(C.Structure):
    """moe_slot_table (include/moe_offload.h)."""
    _fields_ = [("slot_of", C.c_void_p), ("slot_expert", C.c_void_p), ("stamp", C.c_void_p),
                ("step", C.c_void_p), ("n_experts", C.c_int32), ("cap", C.c_int32),
                ("next_slot_of", C.c_void_p), ("next_slot_expert", C.c_void_p),
                ("next_stamp", C.c_void_p), ("next_step", C.c_void_p)]


_vp, _i32, _i64, _sz = C.c_void_p, C.c_int32, C.c_int64, C.c_size_t

# name -> (restype, argtypes); every entry point of include/moe_offload.h
SIGNATURES = {
    "moe_last_error": (C.c_char_p, []),
    "moe_version": (C.c_char_p, []),
    "moe_hip_runtime_path": (C.c_char_p, []),
    "moe_host_alloc": (C.c_int, [C.POINTER(_vp), _sz, C.c_int]),
    "moe_host_free": (C.c_int, [_vp]),
    "moe_device_ptr_of": (C.c_int, [_vp, C.POINTER(_vp)]),
    "moe_slots_init": (C.c_int, [_vp, _i32, _vp, _vp, _i32, _vp, _vp]),
    "moe_resolve_slots": (C.c_int, [_vp, _i32, _i32, _vp, _i32, _vp, _vp, _i32, _vp, _vp, _vp,
                                    _vp, _vp, _vp, _vp]),
    "moe_fetch": (C.c_int, [C.POINTER(FetchPair), _i32, _vp, _vp, _vp, _i32, _i32, _vp]),
    "moe_router_topk": (C.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _i32,
                                  _vp, _i32, _vp]),
    "moe_route_resolve": (C.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp,
                                    _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "moe_route_fetch": (C.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp,
                                  _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                                  C.POINTER(FetchPair), _i32, _i32, _vp]),
    "moe_route_fetch_ffn": (C.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp,
                                      _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                      _vp, C.c_int64, _i32, _i32, C.POINTER(SharedExpert), _vp,
                                      _vp, _vp, _sz, _vp]),
    "moe_route_fetch_ffn_uncached": (C.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp,
                                               _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                               C.c_int64, _i32, _i32, C.POINTER(SharedExpert),
                                               _vp, _vp, _vp, _sz, _vp]),
    "moe_fetch_ffn": (C.c_int, [C.POINTER(FetchPair), _i32, _vp, _vp, _vp, _i32, _i32, _vp,
                                _vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _i32,
                                C.POINTER(ExpertStrides), _vp, _vp, _vp, _sz, _vp]),
    "moe_fp8_moe_workspace": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "moe_fp8_moe_forward": (C.c_int, [_vp, _vp, _i32, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp,
                                      _i32, _i32, _i32, _vp, _vp, _sz, _vp]),
    "moe_fp8_moe_forward_ex": (C.c_int, [_vp, _vp, _i32, _vp, _i32, _i32, _i32, _vp, _vp, _vp,
                                         _vp, _i32, _i32, _i32, C.POINTER(ExpertStrides), _vp,
                                         _vp, _vp, _sz, _i32, _vp]),
    "moe_router_fp8_moe_forward": (C.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp,
                                             _vp, _vp, _vp, _vp, _vp, _i32,
                                             C.POINTER(ExpertStrides), _vp, _vp, _vp, _sz, _vp]),
    "moe_fp8_moe_forward_noalloc": (C.c_int, [_vp, _vp, _i32, _vp, _i32, _i32, _i32, _vp, _vp,
                                              _vp, _vp, _i32, _i32, _i32,
                                              C.POINTER(ExpertStrides), _vp, _vp, _i32, _vp]),
    "moe_permute": (C.c_int, [_vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "moe_unpermute": (C.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "moe_unique_inverse": (C.c_int, [_vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "moe_gather_plan": (C.c_int, [_vp, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _vp]),
    "moe_shared_gate_up": (C.c_int, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp]),
    "moe_shared_down": (C.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "moe_all_finite": (C.c_int, [_vp, _i32, _i64, _vp, _vp]),
    "moe_e4m3_check": (C.c_int, [C.c_uint32, C.c_uint32, _vp, _vp]),
    "moe_silu_check": (C.c_int, [_vp, _vp, _vp, C.c_uint32, _vp]),
    "moe_stream_read": (C.c_int, [_vp, _i64, _i32, _vp, _vp]),
    "moe_time_fused_launch": (C.c_int, [_vp, _vp]),
    "moe_linear_bf16": (C.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _vp, _i32, _vp]),
    "moe_resolve_fetch_ffn": (C.c_int, [_vp, _i32, _i32, C.POINTER(SlotTable), _vp, _vp, _vp, _vp,
                                        _vp, C.POINTER(FetchPair), _i32, _i32, _vp, _vp, _i32, _vp,
                                        _vp, _vp, _vp, _i32, _i32, C.POINTER(ExpertStrides), _vp,
                                        _vp, _vp, _sz, _vp]),
    "moe_codec_histogram": (C.c_int, [_vp, _i64, _i64, _i64, _vp, _i32]),
    "moe_codec_bound": (_i64, [_i64, _i64]),
    "moe_codec_encode": (_i64, [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _i32]),
    "moe_codec_table": (C.c_int, [_vp, _vp]),
    "moe_fetch_coded": (C.c_int, [_vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _i32, _vp, _i64,
                                  _i32, _vp]),
    "moe_route_fetch_coded": (C.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp,
                                        _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                        _vp, _vp, _i64, _i64, _vp, _vp, _i64, _i32, _vp]),
    "moe_fp8_moe_block_workspace": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "moe_fp8_moe_block_forward": (C.c_int, [_vp, _vp, _i32, _vp, _i32, _i32, _i32, _vp, _vp, _vp,
                                            _vp, _i32, _i32, _i32, C.POINTER(ExpertStrides),
                                            C.POINTER(SharedExpert), _vp, _vp, _vp, _sz, _i32,
                                            _vp]),
}


def declared_symbols() -> list[str]:
    """Every function declared in include/moe_offload.h (parsed from the text)."""
    import re
    hdr = (HERE.parent / "include" / "moe_offload.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\**\s+\**(moe_[a-z_0-9]+)\(", hdr,
                                 flags=re.M)))


class NativeError(RuntimeError):
    pass


class Native:
    """Thin typed wrapper over the C ABI.  Tensor arguments are passed by
    data_ptr(); every call is enqueued on torch's current stream."""

    def __init__(self, cdll: C.CDLL):
        self.cdll = cdll
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(cdll, name)
            fn.restype = res
            fn.argtypes = args

    # ------------------------------------------------------------ helpers
    def _check(self, rc: int, what: str) -> None:
        if rc != 0:
            msg = self.cdll.moe_last_error().decode(errors="replace")
            raise NativeError(f"{what} failed ({rc}): {msg}")

    @staticmethod
    def stream() -> int:
        import torch
        return torch.cuda.current_stream().cuda_stream

    @staticmethod
    def _ptr(t) -> int | None:
        return None if t is None else t.data_ptr()

    @staticmethod
    def _on_gpu(what: str, *tensors) -> None:
        """Every tensor argument must live on one GPU: a host address handed
        to a kernel would fault the device, so it is refused here."""
        dev = None
        for t in tensors:
            if t is None:
                continue
            if not t.is_cuda:
                raise ValueError(f"{what}: every tensor argument must be on the GPU, "
                                 f"got one on {t.device}")
            if dev is None:
                dev = t.device
            elif t.device != dev:
                raise ValueError(f"{what}: tensor arguments on {dev} and {t.device}")

    @staticmethod
    def _dtype_code(t) -> int:
        import torch
        codes = {torch.int32: MOE_I32, torch.int64: MOE_I64, torch.float32: MOE_F32,
                 torch.bfloat16: MOE_BF16}
        if t.dtype not in codes:
            raise ValueError(f"no library dtype code for {t.dtype}")
        return codes[t.dtype]

    @staticmethod
    def _buf(what: str, name: str, t, n: int, *dtypes) -> None:
        """Buffer `name` of `what` (None allowed) must be a contiguous tensor
        of at least n elements of one of `dtypes`.  The kernels index it by
        the sizes passed beside it, so a shorter or differently typed buffer
        would be read or written past its end on the device."""
        if t is None:
            return
        if dtypes and t.dtype not in dtypes:
            want = " or ".join(str(d).replace("torch.", "") for d in dtypes)
            raise ValueError(f"{what}: {name} must be {want}, got "
                             f"{str(t.dtype).replace('torch.', '')}")
        if not t.is_contiguous():
            raise ValueError(f"{what}: {name} must be contiguous")
        if t.numel() < n:
            raise ValueError(f"{what}: {name} holds {t.numel()} elements, needs {n}")

    def _slot_bufs(self, what, slot_of, n_experts, slot_expert, stamp, step, out_slot, k,
                   fetch_slot, fetch_expert, nmiss, stats) -> None:
        """The slot table and the per-call outputs of the resolve kernels."""
        import torch
        i32, i64 = torch.int32, torch.int64
        cap = slot_expert.numel()
        for name, t, n, dt in (("slot_of", slot_of, n_experts, i32),
                               ("slot_expert", slot_expert, cap, i32),
                               ("stamp", stamp, cap, i64), ("step", step, 1, i64),
                               ("out_slot", out_slot, k, i32),
                               ("fetch_slot", fetch_slot, k, i32),
                               ("fetch_expert", fetch_expert, k, i32),
                               ("nmiss", nmiss, 1, i32), ("stats", stats, 2, i64)):
            self._buf(what, name, t, n, dt)

    def _router_bufs(self, what, x, w, bias, logits, tokens, top_k) -> tuple[int, int]:
        """x [tokens, H] and w [E, H] bf16, bias f32 [E], logits f32
        [tokens, E]; returns (H, E)."""
        import torch
        if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
            raise ValueError(f"{what}: x [T, H] and w [E, H] must share H")
        H, E = x.shape[1], w.shape[0]
        self._buf(what, "x", x, x.numel(), torch.bfloat16)
        self._buf(what, "w", w, w.numel(), torch.bfloat16)
        self._buf(what, "bias", bias, E, torch.float32)
        self._buf(what, "logits", logits, tokens * E, torch.float32)
        return H, E

    def version(self) -> str:
        return self.cdll.moe_version().decode()

    def hip_runtime_path(self) -> str:
        return self.cdll.moe_hip_runtime_path().decode()

    # ------------------------------------------------------------ host pool
    def host_alloc(self, nbytes: int, noncoherent: bool = False) -> int:
        p = C.c_void_p()
        self._check(self.cdll.moe_host_alloc(C.byref(p), nbytes, 1 if noncoherent else 0),
                    "moe_host_alloc")
        return p.value

    def host_free(self, ptr: int) -> None:
        self._check(self.cdll.moe_host_free(ptr), "moe_host_free")

    def host_buffer(self, nbytes: int, noncoherent: bool = False, on_free=()):
        """(address, uint8 array) of `nbytes` of page-locked, device-mapped host
        memory (moe_host_alloc).  The memory belongs to its views: it is
        freed when the last numpy array or torch.from_numpy tensor over it is
        collected, after `on_free(lo, hi)` of each hook (callers drop cached
        answers about the range there).  Memory still held when the
        interpreter exits is left to the process's end: no HIP call is made
        while the runtime may be shutting down."""
        ptr = self.host_alloc(nbytes, noncoherent=noncoherent)
        buf = (C.c_uint8 * nbytes).from_address(ptr)
        fin = weakref.finalize(buf, _free_host_buffer, self, ptr, nbytes, tuple(on_free))
        fin.atexit = False
        return ptr, np.ctypeslib.as_array(buf)

    def device_ptr_of(self, host_ptr: int) -> int:
        d = C.c_void_p()
        self._check(self.cdll.moe_device_ptr_of(host_ptr, C.byref(d)), "moe_device_ptr_of")
        return d.value

    def is_page_locked(self, t) -> bool:
        """Whether tensor t's storage is page-locked host memory, as the HIP
        runtime sees it.  torch's Tensor.is_pinned() answers False for every
        tensor until torch itself has initialised the GPU, which a process
        that only allocated through this library has not."""
        if t.device.type != "cpu" or t.numel() == 0:
            return False
        d = C.c_void_p()
        return self.cdll.moe_device_ptr_of(t.data_ptr(), C.byref(d)) == 0

    # ------------------------------------------------------------ slots
    def slots_init(self, slot_of, slot_expert, stamp, step) -> None:
        import torch
        self._on_gpu("moe_slots_init", slot_of, slot_expert, stamp, step)
        self._buf("moe_slots_init", "slot_of", slot_of, 1, torch.int32)
        self._buf("moe_slots_init", "slot_expert", slot_expert, 1, torch.int32)
        self._buf("moe_slots_init", "stamp", stamp, slot_expert.numel(), torch.int64)
        self._buf("moe_slots_init", "step", step, 1, torch.int64)
        self._check(self.cdll.moe_slots_init(slot_of.data_ptr(), slot_of.numel(),
                                             slot_expert.data_ptr(), stamp.data_ptr(),
                                             slot_expert.numel(), step.data_ptr(), self.stream()),
                    "moe_slots_init")

    def resolve_slots(self, ids, slot_of, slot_expert, stamp, step, out_slot, fetch_slot,
                      fetch_expert, nmiss, stats=None) -> None:
        import torch
        self._on_gpu("moe_resolve_slots", ids, slot_of, slot_expert, stamp, step, out_slot,
                     fetch_slot, fetch_expert, nmiss, stats)
        self._buf("moe_resolve_slots", "ids", ids, 1, torch.int32, torch.int64)
        self._slot_bufs("moe_resolve_slots", slot_of, slot_of.numel(), slot_expert, stamp, step,
                        out_slot, ids.numel(), fetch_slot, fetch_expert, nmiss, stats)
        self._check(self.cdll.moe_resolve_slots(
            ids.data_ptr(), self._dtype_code(ids), ids.numel(), slot_of.data_ptr(),
            slot_of.numel(), slot_expert.data_ptr(), stamp.data_ptr(), slot_expert.numel(),
            step.data_ptr(), out_slot.data_ptr(), fetch_slot.data_ptr(), fetch_expert.data_ptr(),
            nmiss.data_ptr(), self._ptr(stats), self.stream()), "moe_resolve_slots")

    # ------------------------------------------------------------ fetch
    def fetch(self, pairs, fetch_expert, fetch_slot, nmiss, max_jobs: int,
              blocks_per_job: int) -> None:
        """pairs: [(src_device_addr, dst_device_addr, bytes_per_record[, tile_k]), ...]

        tile_k = K > 0 writes each record, a row-major [rows, K] e4m3 matrix on
        the host, to the cache in MFMA tile order; 0 (the default) copies bytes."""
        import torch
        self._on_gpu("moe_fetch", fetch_expert, fetch_slot, nmiss)
        self._buf("moe_fetch", "fetch_expert", fetch_expert, max_jobs, torch.int32)
        self._buf("moe_fetch", "fetch_slot", fetch_slot, max_jobs, torch.int32)
        self._buf("moe_fetch", "nmiss", nmiss, 1, torch.int32)
        arr = (FetchPair * len(pairs))(*[FetchPair(*((tuple(p) + (0,))[:4])) for p in pairs])
        self._check(self.cdll.moe_fetch(arr, len(pairs), fetch_expert.data_ptr(),
                                        fetch_slot.data_ptr(), nmiss.data_ptr(), max_jobs,
                                        blocks_per_job, self.stream()), "moe_fetch")

    # ------------------------------------------------------------ router
    @staticmethod
    def _logit_code(logit_dtype: str) -> int:
        codes = {"bf16": MOE_BF16, "f32": MOE_F32}
        if logit_dtype not in codes:
            raise ValueError(f"logit_dtype must be 'bf16' or 'f32', got {logit_dtype!r}")
        return codes[logit_dtype]

    def router_topk(self, x, w, bias, top_k: int, logits, ids, weights,
                    logit_dtype: str = "bf16") -> None:
        """logits = x . W^T rounded to logit_dtype ('bf16': the bf16 gate's
        output, or 'f32'), + bias; top-k, softmax over the picks."""
        import torch
        self._on_gpu("moe_router_topk", x, w, bias, logits, ids, weights)
        T = x.shape[0]
        H, E = self._router_bufs("moe_router_topk", x, w, bias, logits, T, top_k)
        self._buf("moe_router_topk", "ids", ids, T * top_k, torch.int32, torch.int64)
        self._buf("moe_router_topk", "weights", weights, T * top_k, torch.float32, torch.bfloat16)
        self._check(self.cdll.moe_router_topk(
            x.data_ptr(), w.data_ptr(), self._ptr(bias), self._logit_code(logit_dtype), T, H, E,
            top_k, logits.data_ptr(),
            ids.data_ptr(), self._dtype_code(ids), weights.data_ptr(), self._dtype_code(weights),
            self.stream()), "moe_router_topk")

    def route_resolve(self, x, w, bias, top_k: int, logits, ids, weights, slot_of, slot_expert,
                      stamp, step, out_slot, fetch_slot, fetch_expert, nmiss, stats=None,
                      logit_dtype: str = "bf16") -> None:
        """Router + slot resolve of one token (ids int32, weights float32)."""
        if x.shape[0] != 1:
            raise ValueError("route_resolve takes exactly one token")
        import torch
        self._on_gpu("moe_route_resolve", x, w, bias, logits, ids, weights, slot_of, slot_expert,
                     stamp, step, out_slot, fetch_slot, fetch_expert, nmiss, stats)
        H, E = self._router_bufs("moe_route_resolve", x, w, bias, logits, 1, top_k)
        self._buf("moe_route_resolve", "ids", ids, top_k, torch.int32)
        self._buf("moe_route_resolve", "weights", weights, top_k, torch.float32)
        self._slot_bufs("moe_route_resolve", slot_of, E, slot_expert, stamp, step, out_slot,
                        top_k, fetch_slot, fetch_expert, nmiss, stats)
        self._check(self.cdll.moe_route_resolve(
            x.data_ptr(), w.data_ptr(), self._ptr(bias), self._logit_code(logit_dtype), H, E,
            top_k, logits.data_ptr(),
            ids.data_ptr(), weights.data_ptr(), slot_of.data_ptr(), slot_expert.data_ptr(),
            stamp.data_ptr(), slot_expert.numel(), step.data_ptr(), out_slot.data_ptr(),
            fetch_slot.data_ptr(), fetch_expert.data_ptr(), nmiss.data_ptr(), self._ptr(stats),
            self.stream()), "moe_route_resolve")

    def route_fetch(self, x, w, bias, top_k: int, logits, ids, weights, slot_of, slot_expert,
                    stamp, step, out_slot, fetch_slot, fetch_expert, nmiss, pairs,
                    blocks_per_job: int, stats=None, logit_dtype: str = "bf16") -> None:
        """Router + slot resolve + fetch of the misses, one token, on a
        double-buffered table: slot_of [2, E], slot_expert and stamp [2, C]
        (buffer 0 set up by slots_init; after a call leaving step = s the
        table is buffer s & 1).  pairs as for fetch()."""
        if x.shape[0] != 1:
            raise ValueError("route_fetch takes exactly one token")
        if slot_of.dim() != 2 or slot_of.shape[0] != 2 or slot_expert.dim() != 2 \
                or slot_expert.shape[0] != 2 or tuple(stamp.shape) != tuple(slot_expert.shape):
            raise ValueError("route_fetch takes double-buffered tables: slot_of [2, E], "
                             "slot_expert and stamp [2, C]")
        import torch
        self._on_gpu("moe_route_fetch", x, w, bias, logits, ids, weights, slot_of, slot_expert,
                     stamp, step, out_slot, fetch_slot, fetch_expert, nmiss, stats)
        H, E = self._router_bufs("moe_route_fetch", x, w, bias, logits, 1, top_k)
        if slot_of.shape[1] != E:
            raise ValueError(f"slot_of [2, {slot_of.shape[1]}] does not match {E} experts")
        self._buf("moe_route_fetch", "ids", ids, top_k, torch.int32)
        self._buf("moe_route_fetch", "weights", weights, top_k, torch.float32)
        self._slot_bufs("moe_route_fetch", slot_of, 2 * E, slot_expert, stamp, step, out_slot,
                        top_k, fetch_slot, fetch_expert, nmiss, stats)
        arr = (FetchPair * len(pairs))(*[FetchPair(*((tuple(p) + (0,))[:4])) for p in pairs])
        self._check(self.cdll.moe_route_fetch(
            x.data_ptr(), w.data_ptr(), self._ptr(bias), self._logit_code(logit_dtype), H, E,
            top_k, logits.data_ptr(), ids.data_ptr(), weights.data_ptr(), slot_of.data_ptr(),
            slot_expert.data_ptr(), stamp.data_ptr(), slot_expert.shape[1], step.data_ptr(),
            out_slot.data_ptr(), fetch_slot.data_ptr(), fetch_expert.data_ptr(), nmiss.data_ptr(),
            self._ptr(stats), arr, len(pairs), blocks_per_job, self.stream()), "moe_route_fetch")

    def route_fetch_ffn(self, x, w, bias, top_k: int, logits, ids, weights, slot_of,
                        slot_expert, stamp, step, out_slot, fetch_slot, fetch_expert, nmiss,
                        pool_dev_ptr: int, cache, inter: int, blocks_per_job: int, out,
                        workspace, residual=None, stats=None, logit_dtype: str = "bf16",
                        shared=None) -> None:
        """The decode step's MoE layer of one token (moe_route_fetch_ffn):
        route_fetch's router, resolve and miss fetch from the packed pool at
        device address pool_dev_ptr into cache (uint8 [cap, record_bytes]),
        then the expert FFN on the slots; out [1, H] bf16 = residual + MoE(x).
        shared = (w_gate [Is, H], w_up [Is, H], w_down [H, Is], w_sgate [H])
        bf16 makes it the MoE block (fp8_moe_block_forward's output)."""
        import torch
        if x.shape[0] != 1:
            raise ValueError("route_fetch_ffn takes exactly one token")
        if slot_of.dim() != 2 or slot_of.shape[0] != 2 or slot_expert.dim() != 2 \
                or slot_expert.shape[0] != 2 or tuple(stamp.shape) != tuple(slot_expert.shape):
            raise ValueError("route_fetch_ffn takes double-buffered tables: slot_of [2, E], "
                             "slot_expert and stamp [2, C]")
        what = "moe_route_fetch_ffn"
        self._on_gpu(what, x, w, bias, logits, ids, weights, slot_of, slot_expert, stamp, step,
                     out_slot, fetch_slot, fetch_expert, nmiss, stats, cache, out, workspace,
                     residual)
        H, E = self._router_bufs(what, x, w, bias, logits, 1, top_k)
        if slot_of.shape[1] != E:
            raise ValueError(f"slot_of [2, {slot_of.shape[1]}] does not match {E} experts")
        C_ = slot_expert.shape[1]
        self._buf(what, "ids", ids, top_k, torch.int32)
        self._buf(what, "weights", weights, top_k, torch.float32)
        self._slot_bufs(what, slot_of, 2 * E, slot_expert, stamp, step, out_slot, top_k,
                        fetch_slot, fetch_expert, nmiss, stats)
        if cache.dim() != 2 or cache.dtype != torch.uint8 or not cache.is_contiguous() \
                or cache.shape[0] < C_:
            raise ValueError(f"{what}: cache must be contiguous uint8 [>= {C_}, record_bytes]")
        se = self._ffn_tail(what, x, H, out, residual, workspace, shared)
        self._check(self.cdll.moe_route_fetch_ffn(
            x.data_ptr(), w.data_ptr(), self._ptr(bias), self._logit_code(logit_dtype), H, E,
            top_k, logits.data_ptr(), ids.data_ptr(), weights.data_ptr(), slot_of.data_ptr(),
            slot_expert.data_ptr(), stamp.data_ptr(), C_, step.data_ptr(), out_slot.data_ptr(),
            fetch_slot.data_ptr(), fetch_expert.data_ptr(), nmiss.data_ptr(), self._ptr(stats),
            pool_dev_ptr, cache.data_ptr(), cache.shape[1], inter, blocks_per_job, se,
            self._ptr(residual), out.data_ptr(), workspace.data_ptr(),
            workspace.numel() * workspace.element_size(), self.stream()), what)

    def route_fetch_ffn_uncached(self, x, w, bias, top_k: int, logits, ids, weights, out_slot,
                                 fetch_slot, fetch_expert, nmiss, pool_dev_ptr: int, cache,
                                 inter: int, blocks_per_job: int, out, workspace, residual=None,
                                 stats=None, logit_dtype: str = "bf16", shared=None) -> None:
        """route_fetch_ffn with no cache policy (moe_route_fetch_ffn_uncached):
        every routed expert fetched into cache slot k (its place in the
        top-k) on every call; out_slot = 0..top_k-1, the miss list = ids."""
        import torch
        if x.shape[0] != 1:
            raise ValueError("route_fetch_ffn_uncached takes exactly one token")
        what = "moe_route_fetch_ffn_uncached"
        self._on_gpu(what, x, w, bias, logits, ids, weights, out_slot, fetch_slot, fetch_expert,
                     nmiss, stats, cache, out, workspace, residual)
        H, E = self._router_bufs(what, x, w, bias, logits, 1, top_k)
        i32 = torch.int32
        for name, t, n, dt in (("ids", ids, top_k, i32), ("weights", weights, top_k, torch.float32),
                               ("out_slot", out_slot, top_k, i32),
                               ("fetch_slot", fetch_slot, top_k, i32),
                               ("fetch_expert", fetch_expert, top_k, i32),
                               ("nmiss", nmiss, 1, i32), ("stats", stats, 2, torch.int64)):
            self._buf(what, name, t, n, dt)
        if cache.dim() != 2 or cache.dtype != torch.uint8 or not cache.is_contiguous():
            raise ValueError(f"{what}: cache must be contiguous uint8 [slots, record_bytes]")
        se = self._ffn_tail(what, x, H, out, residual, workspace, shared)
        self._check(self.cdll.moe_route_fetch_ffn_uncached(
            x.data_ptr(), w.data_ptr(), self._ptr(bias), self._logit_code(logit_dtype), H, E,
            top_k, logits.data_ptr(), ids.data_ptr(), weights.data_ptr(), cache.shape[0],
            out_slot.data_ptr(), fetch_slot.data_ptr(), fetch_expert.data_ptr(),
            nmiss.data_ptr(), self._ptr(stats), pool_dev_ptr, cache.data_ptr(), cache.shape[1],
            inter, blocks_per_job, se, self._ptr(residual), out.data_ptr(),
            workspace.data_ptr(), workspace.numel() * workspace.element_size(), self.stream()),
            what)

    def _ffn_tail(self, what, x, H, out, residual, workspace, shared):
        """The output, residual and workspace buffers of the fused step, and
        the shared expert (w_gate [Is, H], w_up [Is, H], w_down [H, Is],
        w_sgate [H] bf16, or None) as a moe_shared_expert reference."""
        import torch
        self._buf(what, "out", out, H, torch.bfloat16)
        self._buf(what, "residual", residual, H, torch.bfloat16)
        self._buf(what, "workspace", workspace, 0)
        if shared is None:
            return None
        wg, wu, wd, wsg = shared
        self._on_gpu(what, x, *shared)
        Is = wg.shape[0]
        if wg.shape != (Is, H) or wu.shape != (Is, H) or wd.shape != (H, Is) \
                or wsg.numel() != H:
            raise ValueError(f"{what}: shared expert weights do not match x")
        for name, t in zip(("w_gate", "w_up", "w_down", "w_sgate"), shared):
            self._buf(what, name, t, t.numel(), torch.bfloat16)
        return C.byref(SharedExpert(wg.data_ptr(), wu.data_ptr(), wd.data_ptr(), wsg.data_ptr(),
                                    Is))

    def fetch_ffn(self, pairs, fetch_expert, fetch_slot, nmiss, max_jobs: int,
                  blocks_per_job: int, x, slots, weights, w13, s13, w2, s2, out, workspace,
                  residual=None) -> None:
        """moe_fetch of the four buffers (w13, w2, s13, s2 pairs, w13/w2 in tile
        order) and the expert FFN of one token on the cache slots
        (moe_fetch_ffn); out [1, H] bf16 = residual + MoE(x)."""
        import torch
        what = "moe_fetch_ffn"
        self._on_gpu(what, fetch_expert, fetch_slot, nmiss, x, slots, weights, w13, s13, w2, s2,
                     out, workspace, residual)
        if x.dim() != 2 or x.shape[0] != 1:
            raise ValueError(f"{what} takes exactly one token")
        H = x.shape[1]
        K = slots.numel()
        self._buf(what, "x", x, H, torch.bfloat16)
        self._buf(what, "slots", slots, K, torch.int32)
        self._buf(what, "weights", weights, K, torch.float32, torch.bfloat16)
        for name, t in (("fetch_expert", fetch_expert), ("fetch_slot", fetch_slot)):
            self._buf(what, name, t, max_jobs, torch.int32)
        self._buf(what, "nmiss", nmiss, 1, torch.int32)
        self._buf(what, "out", out, H, torch.bfloat16)
        self._buf(what, "residual", residual, H, torch.bfloat16)
        self._buf(what, "workspace", workspace, 0)
        es = _expert_strides(w13, s13, w2, s2, LAYOUT_TILES)
        arr = (FetchPair * len(pairs))(*[FetchPair(*((tuple(p) + (0,))[:4])) for p in pairs])
        self._check(self.cdll.moe_fetch_ffn(
            arr, len(pairs), fetch_expert.data_ptr(), fetch_slot.data_ptr(), nmiss.data_ptr(),
            max_jobs, blocks_per_job, x.data_ptr(), slots.data_ptr(), weights.data_ptr(),
            self._dtype_code(weights), K, w13.data_ptr(), s13.data_ptr(), w2.data_ptr(),
            s2.data_ptr(), w13.shape[0], H, w2.shape[-1], C.byref(es), self._ptr(residual),
            out.data_ptr(), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
            self.stream()), what)

    def resolve_fetch_ffn(self, ids, table, next_table, out_slot, fetch_slot, fetch_expert,
                          nmiss, pairs, blocks_per_job: int, x, weights, w13, s13, w2, s2, out,
                          workspace, residual=None, stats=None) -> None:
        """The drop-in's decode call in two launches (moe_resolve_fetch_ffn):
        the slot resolve of ids [top_k] on table = (slot_of [E], slot_expert
        [C], stamp [C], step [1]) made by the fetch + gate/up launch itself,
        the next table staged in next_table (the same shapes) and copied
        into `table` by the down launch; out [1, H] bf16 = residual + MoE(x)."""
        import torch
        what = "moe_resolve_fetch_ffn"
        self._on_gpu(what, ids, *table, *next_table, out_slot, fetch_slot, fetch_expert, nmiss,
                     x, weights, w13, s13, w2, s2, out, workspace, residual, stats)
        if x.dim() != 2 or x.shape[0] != 1:
            raise ValueError(f"{what} takes exactly one token")
        H = x.shape[1]
        K = ids.numel()
        slot_of, slot_expert, stamp, step = table
        E, cap = slot_of.numel(), slot_expert.numel()
        self._buf(what, "ids", ids, K, torch.int32, torch.int64)
        self._slot_bufs(what, slot_of, E, slot_expert, stamp, step, out_slot, K, fetch_slot,
                        fetch_expert, nmiss, stats)
        for name, t, ref in zip(("next_slot_of", "next_slot_expert", "next_stamp", "next_step"),
                                next_table, table):
            self._buf(what, name, t, ref.numel(), ref.dtype)
        self._buf(what, "x", x, H, torch.bfloat16)
        self._buf(what, "weights", weights, K, torch.float32, torch.bfloat16)
        self._buf(what, "out", out, H, torch.bfloat16)
        self._buf(what, "residual", residual, H, torch.bfloat16)
        self._buf(what, "workspace", workspace, 0)
        if w13.shape[0] != cap:
            raise ValueError(f"{what}: the cache holds {w13.shape[0]} slots, the table {cap}")
        es = _expert_strides(w13, s13, w2, s2, LAYOUT_TILES)
        tab = SlotTable(slot_of.data_ptr(), slot_expert.data_ptr(), stamp.data_ptr(),
                        step.data_ptr(), E, cap, *(t.data_ptr() for t in next_table))
        arr = (FetchPair * len(pairs))(*[FetchPair(*((tuple(p) + (0,))[:4])) for p in pairs])
        self._check(self.cdll.moe_resolve_fetch_ffn(
            ids.data_ptr(), self._dtype_code(ids), K, C.byref(tab), out_slot.data_ptr(),
            fetch_slot.data_ptr(), fetch_expert.data_ptr(), nmiss.data_ptr(), self._ptr(stats),
            arr, len(pairs), blocks_per_job, x.data_ptr(), weights.data_ptr(),
            self._dtype_code(weights), w13.data_ptr(), s13.data_ptr(), w2.data_ptr(),
            s2.data_ptr(), H, w2.shape[-1], C.byref(es), self._ptr(residual), out.data_ptr(),
            workspace.data_ptr(), workspace.numel() * workspace.element_size(), self.stream()),
            what)

    # ------------------------------------------------------------ experts
    def fp8_moe_workspace(self, tokens, top_k, n_experts, hidden, inter) -> int:
        return int(self.cdll.moe_fp8_moe_workspace(tokens, top_k, n_experts, hidden, inter))

    def fp8_moe_forward(self, x, ids, weights, w13, s13, w2, s2, out, workspace,
                        mode: int = 0, residual=None, layout: int = LAYOUT_ROWS) -> None:
        """w13/s13/w2/s2 may be strided along the expert axis (views into a
        packed record pool); every other dimension must be contiguous.
        `layout`: byte order of w13/w2 (LAYOUT_TILES for record views)."""
        self._on_gpu("moe_fp8_moe_forward", x, ids, weights, w13, s13, w2, s2, out, workspace,
                     residual)
        T, H = x.shape
        K = ids.shape[-1]
        n = w13.shape[0]
        inter = w2.shape[-1]
        es = _expert_strides(w13, s13, w2, s2, layout)
        self._check(self.cdll.moe_fp8_moe_forward_ex(
            x.data_ptr(), ids.data_ptr(), self._dtype_code(ids), weights.data_ptr(),
            self._dtype_code(weights), T, K, w13.data_ptr(), s13.data_ptr(), w2.data_ptr(),
            s2.data_ptr(), n, H, inter, C.byref(es), self._ptr(residual), out.data_ptr(),
            workspace.data_ptr(),
            workspace.numel() * workspace.element_size(), mode, self.stream()),
            "moe_fp8_moe_forward")

    def router_fp8_moe_forward(self, x, w_gate, bias, top_k: int, logits, ids, weights, w13,
                               s13, w2, s2, out, workspace, residual=None,
                               logit_dtype: str = "bf16", layout: int = LAYOUT_ROWS) -> None:
        """The router and expert FFN of 1-16 tokens over resident experts
        (moe_router_fp8_moe_forward): logits [T, E] f32, ids [T, top_k] int32
        and weights [T, top_k] f32 written; out [T, H] = residual + MoE(x),
        as router_topk followed by fp8_moe_forward(mode=1)."""
        import torch
        what = "moe_router_fp8_moe_forward"
        self._on_gpu(what, x, w_gate, bias, logits, ids, weights, w13, s13, w2, s2, out,
                     workspace, residual)
        if x.dim() != 2:
            raise ValueError(f"{what}: x must be [T, H]")
        T = x.shape[0]
        H, E = self._router_bufs(what, x, w_gate, bias, logits, T, top_k)
        if w13.shape[0] != E:
            raise ValueError(f"{what}: {w13.shape[0]} experts' weights for a {E}-expert router")
        self._buf(what, "ids", ids, T * top_k, torch.int32)
        self._buf(what, "weights", weights, T * top_k, torch.float32)
        self._buf(what, "out", out, T * H, torch.bfloat16)
        self._buf(what, "residual", residual, T * H, torch.bfloat16)
        es = _expert_strides(w13, s13, w2, s2, layout)
        self._check(self.cdll.moe_router_fp8_moe_forward(
            x.data_ptr(), w_gate.data_ptr(), self._ptr(bias), self._logit_code(logit_dtype), T,
            H, E, top_k, logits.data_ptr(), ids.data_ptr(), weights.data_ptr(), w13.data_ptr(),
            s13.data_ptr(), w2.data_ptr(), s2.data_ptr(), w2.shape[-1], C.byref(es),
            self._ptr(residual), out.data_ptr(), workspace.data_ptr(),
            workspace.numel() * workspace.element_size(), self.stream()), what)

    def fp8_moe_forward_noalloc(self, x, ids, weights, w13, s13, w2, s2, out, mode: int = 0,
                                residual=None, layout: int = LAYOUT_ROWS) -> None:
        """fp8_moe_forward with the library's per-GPU scratch array as the
        workspace: allocates nothing (moe_fp8_moe_forward_noalloc)."""
        self._on_gpu("moe_fp8_moe_forward_noalloc", x, ids, weights, w13, s13, w2, s2, out,
                     residual)
        T, H = x.shape
        K = ids.shape[-1]
        n = w13.shape[0]
        inter = w2.shape[-1]
        es = _expert_strides(w13, s13, w2, s2, layout)
        self._check(self.cdll.moe_fp8_moe_forward_noalloc(
            x.data_ptr(), ids.data_ptr(), self._dtype_code(ids), weights.data_ptr(),
            self._dtype_code(weights), T, K, w13.data_ptr(), s13.data_ptr(), w2.data_ptr(),
            s2.data_ptr(), n, H, inter, C.byref(es), self._ptr(residual), out.data_ptr(), mode,
            self.stream()), "moe_fp8_moe_forward_noalloc")

    def fp8_moe_block_workspace(self, tokens, top_k, n_experts, hidden, inter,
                                shared_inter) -> int:
        return int(self.cdll.moe_fp8_moe_block_workspace(tokens, top_k, n_experts, hidden, inter,
                                                         shared_inter))

    def fp8_moe_block_forward(self, x, ids, weights, w13, s13, w2, s2, shared, out, workspace,
                              mode: int = 0, residual=None, layout: int = LAYOUT_ROWS) -> None:
        """The MoE block: routed experts plus the gated shared expert,
        shared = (w_gate [Is, H], w_up [Is, H], w_down [H, Is], w_sgate [H]) bf16;
        out = residual + (routed + sigmoid-gated shared), each sum rounded to bf16."""
        self._on_gpu("moe_fp8_moe_block_forward", x, ids, weights, w13, s13, w2, s2, *shared, out,
                     workspace, residual)
        T, H = x.shape
        K = ids.shape[-1]
        n = w13.shape[0]
        inter = w2.shape[-1]
        wg, wu, wd, wsg = shared
        Is = wg.shape[0]
        if wg.shape != (Is, H) or wu.shape != (Is, H) or wd.shape != (H, Is) or wsg.numel() != H:
            raise ValueError("shared expert weights do not match x")
        es = _expert_strides(w13, s13, w2, s2, layout)
        se = SharedExpert(wg.data_ptr(), wu.data_ptr(), wd.data_ptr(), wsg.data_ptr(), Is)
        self._check(self.cdll.moe_fp8_moe_block_forward(
            x.data_ptr(), ids.data_ptr(), self._dtype_code(ids), weights.data_ptr(),
            self._dtype_code(weights), T, K, w13.data_ptr(), s13.data_ptr(), w2.data_ptr(),
            s2.data_ptr(), n, H, inter, C.byref(es), C.byref(se), self._ptr(residual),
            out.data_ptr(), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
            mode, self.stream()), "moe_fp8_moe_block_forward")

    # ------------------------------------------------------------ permute
    def permute(self, ids, n_experts: int, counts, offsets, sorted_pairs, pair_pos) -> None:
        import torch
        self._on_gpu("moe_permute", ids, counts, offsets, sorted_pairs, pair_pos)
        T, K = ids.shape
        self._buf("moe_permute", "ids", ids, T * K, torch.int32, torch.int64)
        for name, t, n in (("counts", counts, n_experts), ("offsets", offsets, n_experts + 1),
                           ("sorted_pairs", sorted_pairs, T * K), ("pair_pos", pair_pos, T * K)):
            self._buf("moe_permute", name, t, n, torch.int32)
        self._check(self.cdll.moe_permute(ids.data_ptr(), self._dtype_code(ids), T, K, n_experts,
                                          counts.data_ptr(), offsets.data_ptr(),
                                          sorted_pairs.data_ptr(), pair_pos.data_ptr(),
                                          self.stream()), "moe_permute")

    def unique_inverse(self, ids, n_experts: int, counts, n_unique, uniq, rank_of,
                       inverse) -> None:
        import torch
        self._on_gpu("moe_unique_inverse", ids, counts, n_unique, uniq, rank_of, inverse)
        T, K = ids.shape
        self._buf("moe_unique_inverse", "ids", ids, T * K, torch.int32, torch.int64)
        for name, t, n in (("counts", counts, n_experts), ("n_unique", n_unique, 1),
                           ("uniq", uniq, n_experts), ("rank_of", rank_of, n_experts),
                           ("inverse", inverse, T * K)):
            self._buf("moe_unique_inverse", name, t, n, torch.int32)
        self._check(self.cdll.moe_unique_inverse(
            ids.data_ptr(), self._dtype_code(ids), T, K, n_experts, counts.data_ptr(),
            n_unique.data_ptr(), uniq.data_ptr(), rank_of.data_ptr(), inverse.data_ptr(),
            self.stream()), "moe_unique_inverse")

    def gather_plan(self, uniq, n_unique, slot_of, cap: int, host_expert, host_dst, n_host,
                    cache_src, cache_dst, n_cache, stats=None) -> None:
        import torch
        self._on_gpu("moe_gather_plan", uniq, n_unique, slot_of, host_expert, host_dst, n_host,
                     cache_src, cache_dst, n_cache, stats)
        E = uniq.numel()
        for name, t, n in (("uniq", uniq, E), ("n_unique", n_unique, 1),
                           ("slot_of", slot_of, E if cap > 0 else 0),
                           ("host_expert", host_expert, E), ("host_dst", host_dst, E),
                           ("n_host", n_host, 1), ("cache_src", cache_src, E),
                           ("cache_dst", cache_dst, E), ("n_cache", n_cache, 1)):
            self._buf("moe_gather_plan", name, t, n, torch.int32)
        self._buf("moe_gather_plan", "stats", stats, 2, torch.int64)
        self._check(self.cdll.moe_gather_plan(
            uniq.data_ptr(), n_unique.data_ptr(), self._ptr(slot_of), uniq.numel(), cap,
            host_expert.data_ptr(), host_dst.data_ptr(), n_host.data_ptr(), cache_src.data_ptr(),
            cache_dst.data_ptr(), n_cache.data_ptr(), self._ptr(stats), self.stream()),
            "moe_gather_plan")

    def shared_gate_up(self, x, w_gate, w_up, w_sgate, act, sig) -> None:
        """Shared expert, first half: act [T, Is] bf16 and the sigmoid gate
        sig [T] f32 from x [T, H] bf16 (weights bf16, row-major)."""
        T, H = x.shape
        Is = w_gate.shape[0]
        if w_gate.shape != (Is, H) or w_up.shape != (Is, H) or w_sgate.numel() != H:
            raise ValueError("shared expert weights do not match x")
        if act.shape != (T, Is) or sig.numel() < T:
            raise ValueError("shared expert scratch too small")
        self._on_gpu("moe_shared_gate_up", x, w_gate, w_up, w_sgate, act, sig)
        self._check(self.cdll.moe_shared_gate_up(
            x.data_ptr(), w_gate.data_ptr(), w_up.data_ptr(), w_sgate.data_ptr(), T, H, Is,
            act.data_ptr(), sig.data_ptr(), self.stream()), "moe_shared_gate_up")

    def shared_down(self, act, sig, w_down, out, routed=None, residual=None) -> None:
        """Shared expert, second half: out = residual + (routed + sig * act W_down^T),
        each term rounded to bf16 (routed / residual optional)."""
        T, Is = act.shape
        H = w_down.shape[0]
        if w_down.shape != (H, Is) or out.shape != (T, H):
            raise ValueError("shared expert down weights do not match")
        for t in (routed, residual):
            if t is not None and t.shape != (T, H):
                raise ValueError("routed / residual must be [T, H]")
        self._on_gpu("moe_shared_down", act, sig, w_down, out, routed, residual)
        self._check(self.cdll.moe_shared_down(
            act.data_ptr(), sig.data_ptr(), w_down.data_ptr(), T, H, Is, self._ptr(routed),
            self._ptr(residual), out.data_ptr(), self.stream()), "moe_shared_down")

    def all_finite(self, x, flag) -> None:
        """flag[0] (int32, device) = 1 if every element of x (f32 or bf16) is finite."""
        import torch
        self._on_gpu("moe_all_finite", x, flag)
        self._buf("moe_all_finite", "x", x, x.numel(), torch.float32, torch.bfloat16)
        self._buf("moe_all_finite", "flag", flag, 1, torch.int32)
        self._check(self.cdll.moe_all_finite(x.data_ptr(), self._dtype_code(x), x.numel(),
                                             flag.data_ptr(), self.stream()), "moe_all_finite")

    def e4m3_check(self, first: int, count: int, mismatches) -> None:
        """Add to mismatches[0] (int64, device) the bit patterns of
        [first, first + count) whose hardware e4m3 encoding differs from the
        software encoder's (moe_e4m3_check)."""
        import torch
        self._on_gpu("moe_e4m3_check", mismatches)
        self._buf("moe_e4m3_check", "mismatches", mismatches, 1, torch.int64)
        self._check(self.cdll.moe_e4m3_check(first, count, mismatches.data_ptr(), self.stream()),
                    "moe_e4m3_check")

    def silu_check(self, g, u, out) -> None:
        """out = the expert kernels' SiLU(g) * u, elementwise on float32
        device tensors of one size (moe_silu_check)."""
        import torch
        if not (g.numel() == u.numel() == out.numel()):
            raise ValueError("g, u and out must have one size")
        for t in (g, u, out):
            if t.dtype != torch.float32 or not t.is_contiguous():
                raise ValueError("g, u and out must be contiguous float32")
        self._on_gpu("moe_silu_check", g, u, out)
        self._check(self.cdll.moe_silu_check(g.data_ptr(), u.data_ptr(), out.data_ptr(),
                                             g.numel(), self.stream()), "moe_silu_check")

    def stream_read(self, src, nbytes: int, workgroups: int, sink, offset: int = 0) -> None:
        """Read nbytes of the device tensor src from byte `offset` once
        (moe_stream_read); sink: device uint32/int32 [>= 1]."""
        import torch
        self._on_gpu("moe_stream_read", src, sink)
        self._buf("moe_stream_read", "sink", sink, 1, torch.int32, torch.uint32)
        if offset < 0 or offset + nbytes > src.numel() * src.element_size():
            raise ValueError("stream_read range past the end of src")
        self._check(self.cdll.moe_stream_read(src.data_ptr() + offset, nbytes, workgroups,
                                               sink.data_ptr(), self.stream()),
                    "moe_stream_read")

    def linear_bf16(self, x, w, out, rows_per_wave: int = 0, x_add=None) -> None:
        """out [T, N] = x [T, K] w^T, w [N, K] bf16 (nn.Linear layout), 1 <= T <= 4
        (moe_linear_bf16); with x_add [T, K] bf16 the product is of x + x_add
        (a bf16 add)."""
        import torch
        what = "moe_linear_bf16"
        self._on_gpu(what, x, w, out, x_add)
        if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
            raise ValueError(f"{what}: x [T, K] and w [N, K] must agree on K")
        T, K = x.shape
        N = w.shape[0]
        self._buf(what, "x", x, T * K, torch.bfloat16)
        self._buf(what, "x_add", x_add, T * K, torch.bfloat16)
        self._buf(what, "w", w, N * K, torch.bfloat16)
        self._buf(what, "out", out, T * N, torch.bfloat16)
        self._check(self.cdll.moe_linear_bf16(x.data_ptr(), self._ptr(x_add), w.data_ptr(), T, K,
                                              N, out.data_ptr(), rows_per_wave, self.stream()),
                    what)

    def time_fused_launch(self, start, stop) -> None:
        """Arm torch.cuda.Event start/stop (enable_timing=True) around this
        thread's next fused fetch + gate/up launch (moe_time_fused_launch);
        None, None disarms.  start.elapsed_time(stop) is then that kernel's
        own duration.  Not during stream capture."""
        handles = []
        for ev in (start, stop):
            if ev is None:
                handles.append(None)
                continue
            if not ev.cuda_event:
                ev.record()                 # torch creates the HIP event on first use
            handles.append(ev.cuda_event)
        self._check(self.cdll.moe_time_fused_launch(*handles), "moe_time_fused_launch")

    # ------------------------------------------------------------ coded pools
    def codec_histogram(self, records: np.ndarray, fp8_bytes: int, threads: int = 8):
        """Counts of the 16 e4m3 exponent values over the fp8 part of every
        record of records (uint8 [n, record_bytes], host memory)."""
        n, rb = records.shape
        hist = np.zeros(16, dtype=np.uint64)
        self._check(self.cdll.moe_codec_histogram(records.ctypes.data, n, rb, fp8_bytes,
                                                  hist.ctypes.data, threads), "moe_codec_histogram")
        return hist

    def codec_bound(self, record_bytes: int, fp8_bytes: int) -> int:
        return int(self.cdll.moe_codec_bound(record_bytes, fp8_bytes))

    def codec_encode(self, records: np.ndarray, fp8_bytes: int, lengths, dst: np.ndarray,
                     threads: int = 8):
        """Code every record of records into dst (uint8, host); returns
        (bytes used, record offsets int64 [n+1], block offsets uint32 [n, nblk+1])."""
        n, rb = records.shape
        nblk = fp8_bytes // 8192
        ln = np.ascontiguousarray(lengths, dtype=np.uint8)
        rec_off = np.zeros(n + 1, dtype=np.int64)
        blk_off = np.zeros((n, nblk + 1), dtype=np.uint32)
        used = int(self.cdll.moe_codec_encode(records.ctypes.data, n, rb, fp8_bytes,
                                              ln.ctypes.data, dst.ctypes.data, dst.nbytes,
                                              rec_off.ctypes.data, blk_off.ctypes.data, threads))
        if used < 0:
            self._check(used, "moe_codec_encode")
        return used, rec_off, blk_off

    def codec_table(self, lengths) -> np.ndarray:
        ln = np.ascontiguousarray(lengths, dtype=np.uint8)
        lut = np.zeros(4096, dtype=np.uint16)
        self._check(self.cdll.moe_codec_table(ln.ctypes.data, lut.ctypes.data), "moe_codec_table")
        return lut

    def fetch_coded(self, pool_dev_ptr: int, rec_off, blk_off, record_bytes: int, fp8_bytes: int,
                    lut, fetch_expert, fetch_slot, nmiss, max_jobs: int, cache,
                    workgroups: int = 32) -> None:
        """Decode coded records fetch_expert[j] into cache slots fetch_slot[j],
        j < nmiss[0] (device tensors); cache uint8 [slots, >= record_bytes]."""
        import torch
        self._on_gpu("moe_fetch_coded", rec_off, blk_off, lut, fetch_expert, fetch_slot, nmiss,
                     cache)
        self._buf("moe_fetch_coded", "lut", lut, 4096, torch.uint16, torch.int16)
        for name, t in (("fetch_expert", fetch_expert), ("fetch_slot", fetch_slot)):
            self._buf("moe_fetch_coded", name, t, max_jobs, torch.int32)
        self._buf("moe_fetch_coded", "nmiss", nmiss, 1, torch.int32)
        if cache.dim() != 2 or cache.stride(1) != 1 or \
                cache.shape[1] * cache.element_size() < record_bytes:
            raise ValueError("moe_fetch_coded: cache must be [slots, >= record_bytes] with "
                             "contiguous rows")
        self._check(self.cdll.moe_fetch_coded(
            pool_dev_ptr, rec_off.data_ptr(), blk_off.data_ptr(), record_bytes, fp8_bytes,
            lut.data_ptr(), fetch_expert.data_ptr(), fetch_slot.data_ptr(), nmiss.data_ptr(),
            max_jobs, cache.data_ptr(), cache.stride(0) * cache.element_size(), workgroups,
            self.stream()), "moe_fetch_coded")

    def route_fetch_coded(self, x, w, bias, top_k: int, logits, ids, weights, slot_of,
                          slot_expert, stamp, step, out_slot, fetch_slot, fetch_expert, nmiss,
                          pool_dev_ptr: int, rec_off, blk_off, record_bytes: int, fp8_bytes: int,
                          lut, cache, workgroups: int = 32, stats=None,
                          logit_dtype: str = "bf16") -> None:
        """route_fetch for a coded pool (moe_route_fetch_coded): the router,
        the slot resolve on the double-buffered table and the decode of the
        misses' coded records into cache (uint8 [cap, >= record_bytes]), in
        two launches; the outputs those of route_resolve + fetch_coded."""
        import torch
        what = "moe_route_fetch_coded"
        if x.shape[0] != 1:
            raise ValueError("route_fetch_coded takes exactly one token")
        if slot_of.dim() != 2 or slot_of.shape[0] != 2 or slot_expert.dim() != 2 \
                or slot_expert.shape[0] != 2 or tuple(stamp.shape) != tuple(slot_expert.shape):
            raise ValueError("route_fetch_coded takes double-buffered tables: slot_of [2, E], "
                             "slot_expert and stamp [2, C]")
        self._on_gpu(what, x, w, bias, logits, ids, weights, slot_of, slot_expert, stamp, step,
                     out_slot, fetch_slot, fetch_expert, nmiss, stats, rec_off, blk_off, lut,
                     cache)
        H, E = self._router_bufs(what, x, w, bias, logits, 1, top_k)
        if slot_of.shape[1] != E:
            raise ValueError(f"slot_of [2, {slot_of.shape[1]}] does not match {E} experts")
        self._buf(what, "ids", ids, top_k, torch.int32)
        self._buf(what, "weights", weights, top_k, torch.float32)
        self._slot_bufs(what, slot_of, 2 * E, slot_expert, stamp, step, out_slot, top_k,
                        fetch_slot, fetch_expert, nmiss, stats)
        self._buf(what, "lut", lut, 4096, torch.uint16, torch.int16)
        self._buf(what, "rec_off", rec_off, E + 1, torch.int64)
        nblk = fp8_bytes // 8192
        self._buf(what, "blk_off", blk_off, E * (nblk + 1), torch.uint32, torch.int32)
        if cache.dim() != 2 or cache.stride(1) != 1 or \
                cache.shape[1] * cache.element_size() < record_bytes:
            raise ValueError(f"{what}: cache must be [slots, >= record_bytes] with contiguous "
                             "rows")
        if cache.shape[0] < slot_expert.shape[1]:
            raise ValueError(f"{what}: cache has {cache.shape[0]} slots, the table "
                             f"{slot_expert.shape[1]}")
        self._check(self.cdll.moe_route_fetch_coded(
            x.data_ptr(), w.data_ptr(), self._ptr(bias), self._logit_code(logit_dtype), H, E,
            top_k, logits.data_ptr(), ids.data_ptr(), weights.data_ptr(), slot_of.data_ptr(),
            slot_expert.data_ptr(), stamp.data_ptr(), slot_expert.shape[1], step.data_ptr(),
            out_slot.data_ptr(), fetch_slot.data_ptr(), fetch_expert.data_ptr(),
            nmiss.data_ptr(), self._ptr(stats), pool_dev_ptr, rec_off.data_ptr(),
            blk_off.data_ptr(), record_bytes, fp8_bytes, lut.data_ptr(), cache.data_ptr(),
            cache.stride(0) * cache.element_size(), workgroups, self.stream()), what)

    def unpermute(self, y, pair_pos, weights, out) -> None:
        import torch
        self._on_gpu("moe_unpermute", y, pair_pos, weights, out)
        T, K = weights.shape
        H = y.shape[-1]
        self._buf("moe_unpermute", "y", y, T * K * H, torch.float32)
        self._buf("moe_unpermute", "pair_pos", pair_pos, T * K, torch.int32)
        self._buf("moe_unpermute", "weights", weights, T * K, torch.float32, torch.bfloat16)
        self._buf("moe_unpermute", "out", out, T * H, torch.bfloat16)
        self._check(self.cdll.moe_unpermute(y.data_ptr(), pair_pos.data_ptr(),
                                            weights.data_ptr(), self._dtype_code(weights), T, K,
                                            H, out.data_ptr(), self.stream()), "moe_unpermute")


def _torch_hip_runtime() -> str | None:
    """Path of the libamdhip64 torch loaded, from /proc/self/maps."""
    try:
        with open("/proc/self/maps") as fh:
            for line in fh:
                if "libamdhip64.so" in line:
                    return line.split()[-1]
    except OSError:
        pass
    return None


def load(verbose: bool = False):
    """Return the bound library, or None with the reason in last_error().
    Never raises (bin/cppfetch.py:141-179 contract)."""
    global _lib, _err
    if _lib is not None or _err is not None:
        return _lib
    try:
        import torch  # noqa: F401  -- load torch's HIP runtime first
    except Exception as exc:                                   # noqa: BLE001
        _err = f"torch import failed: {type(exc).__name__}: {exc}"
        return None
    if not LIB_PATH.is_file():
        _err = (f"missing {LIB_PATH}; build it with "
                f"`python drama3-offloading_amd/build.py` (needs hipcc)")
        return None
    try:
        cdll = C.CDLL(str(LIB_PATH), mode=C.RTLD_GLOBAL)
        lib = Native(cdll)
    except (OSError, AttributeError) as exc:
        _err = f"{type(exc).__name__}: {exc}"
        return None
    ours = lib.hip_runtime_path()
    theirs = _torch_hip_runtime()
    if theirs and ours and os.path.realpath(ours) != os.path.realpath(theirs):
        _err = (f"libmoeoffload bound HIP runtime {ours} but torch uses {theirs}; "
                f"two HIP runtimes in one process cannot share streams")
        return None
    if verbose:
        print(f"libmoeoffload: {LIB_PATH} ({lib.version()}), HIP runtime {ours}")
    _lib = lib
    return _lib


def last_error() -> str | None:
    return _err


def require() -> Native:
    """The library, or RuntimeError naming why it cannot be used."""
    lib = load()
    if lib is None:
        raise RuntimeError(f"libmoeoffload (HIP kernels) unavailable: {_err}")
    return lib


def reset() -> None:
    """Forget a previous load result (tests)."""
    global _lib, _err
    _lib = None
    _err = None
