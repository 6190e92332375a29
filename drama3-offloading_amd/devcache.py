"""Device-resident expert cache: no host sync, hipGraph capturable.

Drop-in for bin/devcache.py.  Same per-layer state on the experts module,
same function names and the same dispatch, with the two Triton kernels and
the CUDA extension replaced by libmoeoffload's HIP kernels:

  _dc_slot_of[E]      int32  expert -> slot, -1 absent
  _dc_slot_expert[C]  int32  slot -> expert, -1 empty
  _dc_stamp[C]        int64  step at which the slot was last used
  _dc_step[1]         int64  bumped on the device by every resolve
  _dc_w13/_dc_w2/_dc_s13/_dc_s2   the cache buffers, one slot per row
  _dc_tiles           bool   w13/w2 slots in MFMA tile order (new: the
                             fetch writes them so from the row-major host
                             buffers; offload.DEVICE_TILES at init)
  _dc_out/_dc_fslot/_dc_fexp/_dc_nmiss  per-call scratch, preallocated
  _dc_stats[2]        int64  hits, misses counted on the device (new: the
                             reference has no hit counter, bin/devcache.py:274)

Per decode step (rows == 1): `moe_resolve_slots` (one wavefront; decisions
identical to bin/devcache.py:65-98) then one `moe_fetch` launch that copies
every queued miss, all four buffers, from page-locked host memory into its
slot, reading the miss list and count on the device at run time -- so the
captured graph serves different experts on every replay -- then
`fp8_moe_forward` on the whole cache buffer with slot ids (cache_layout
gives the byte order to pass with the cache buffers).  With CODED_POOL
the weights of the misses come from entropy-coded host copies instead
(two `moe_fetch_coded` launches, then the scales raw).  Prefill
(rows != 1) goes to offload.offloaded_forward, as in the reference
(bin/devcache.py:270-271), whose direct mode gathers on the device and
borrows this cache's resident experts without a host sync.
"""
from __future__ import annotations

import sys as _sys

import torch

import hipfetch
from fp8_moe import fp8_moe_forward

EXPERT_BYTES = 3_146_496

# Accepted for drop-in compatibility with --fetch-backend (bin/devcache.py:191):
# every value selects the one HIP fetch kernel.  The reference's two backends
# existed because one was Triton; there is only one implementation here.
FETCH_BACKEND = "hip"
_BACKENDS = ("hip", "cpp", "triton")
_BACKEND_NOTED = False
# Fetch workgroups per job, up to 8 jobs (bin/devcache.py:193).  3 keeps
# ~192 KiB of host reads in flight, about the link's bandwidth-delay product
# (the best of 2, 3, 4, 6 and 8 measured at 1, 3 and 8 misses).
CPP_BLOCKS_PER_JOB = 3
# dev_cached_forward: the slot resolve, the misses' fetch and the expert FFN
# in two launches (moe_resolve_fetch_ffn: every workgroup of the first makes
# the resolve's decisions, the fetch workgroups run a miss's gate/up on its
# rows as they arrive, the second launch forms the output and updates the
# table) instead of a resolve, a fetch and the FFN's two; same output, same
# table.  Applies to tile-ordered caches of raw pools, hidden a multiple of
# 512, top_k <= 16.
FUSED_FFN = True
_dev_ptr_cache: dict[int, int] = {}
# True: init_dev_cache also keeps the layer's w13 and w2 entropy-coded in
# page-locked memory (codec.CodedPool, about 85 % of their size for
# block-scaled fp8 weights) and decode misses are fetched from there,
# decoded on the GPU (moe_fetch_coded; the scales still come raw).  The
# cache receives the same bytes; the link carries fewer.  Costs about 0.5 s
# per layer at init and a second page-locked copy of w13/w2.
CODED_POOL = False


def init_dev_cache(experts, device: torch.device, capacity: int) -> None:
    """Allocate one layer's cache buffers and slot table (bin/devcache.py:138-167).
    The per-call scratch holds 8 ids, the reference's top-k; a model routing
    to more sets experts._dc_kmax to its top-k first."""
    import offload
    lib = hipfetch.require()
    n_experts = experts.num_experts
    if not 1 <= capacity <= 4096:
        raise ValueError(f"capacity must be in [1, 4096], got {capacity}")
    experts._dc_cap = capacity
    experts._dc_slot_of = torch.empty((n_experts,), dtype=torch.int32, device=device)
    experts._dc_slot_expert = torch.empty((capacity,), dtype=torch.int32, device=device)
    # stamps -C..-1 so the first `capacity` misses take slots 0, 1, 2, ...
    experts._dc_stamp = torch.empty((capacity,), dtype=torch.int64, device=device)
    experts._dc_step = torch.empty((1,), dtype=torch.int64, device=device)
    with torch.cuda.device(device):
        lib.slots_init(experts._dc_slot_of, experts._dc_slot_expert, experts._dc_stamp,
                       experts._dc_step)

    def buf(src):
        return torch.zeros((capacity, *src.shape[1:]), dtype=src.dtype, device=device)

    experts._dc_w13 = buf(experts.w13_weight)
    experts._dc_w2 = buf(experts.w2_weight)
    experts._dc_s13 = torch.ones((capacity, *experts.w13_scale_inv.shape[1:]),
                                 dtype=torch.float32, device=device)
    experts._dc_s2 = torch.ones((capacity, *experts.w2_scale_inv.shape[1:]),
                                dtype=torch.float32, device=device)
    # per-call outputs of the resolve live here for good: a captured step
    # reads and writes the same buffers on every replay
    kmax = max(8, getattr(experts, "_dc_kmax", 8))
    experts._dc_out = torch.zeros(kmax, dtype=torch.int32, device=device)
    experts._dc_fslot = torch.zeros(kmax, dtype=torch.int32, device=device)
    experts._dc_fexp = torch.zeros(kmax, dtype=torch.int32, device=device)
    experts._dc_nmiss = torch.zeros(1, dtype=torch.int32, device=device)
    experts._dc_stats = torch.zeros(2, dtype=torch.int64, device=device)
    # the table's next state, staged by the fused decode call's first launch
    # (all of whose workgroups read the table) and copied in by its second
    experts._dc_next = tuple(torch.empty_like(t) for t in (
        experts._dc_slot_of, experts._dc_slot_expert, experts._dc_stamp, experts._dc_step))
    experts._dc_pairs = None
    experts._dc_tiles = bool(offload.DEVICE_TILES)
    experts._dc_coded = _code_weights(experts, device) if CODED_POOL else None


def cache_layout(experts) -> int:
    """hipfetch.LAYOUT_* of the cache's w13/w2 slots, for fp8_moe_forward."""
    return hipfetch.LAYOUT_TILES if getattr(experts, "_dc_tiles", False) else hipfetch.LAYOUT_ROWS


def reset_dev_cache(experts) -> None:
    """Empty an initialised cache in place: same tensors (so a captured graph
    that references them stays valid), table back to its initial state,
    device hit/miss counters cleared.  Slot contents are left as they are;
    an empty slot is never handed out before it is filled."""
    lib = hipfetch.require()
    with torch.cuda.device(experts._dc_slot_of.device):
        lib.slots_init(experts._dc_slot_of, experts._dc_slot_expert, experts._dc_stamp,
                       experts._dc_step)
        experts._dc_stats.zero_()


def _code_weights(experts, device):
    """(w13, w2) of every expert as two coded pools, coding the bytes in the
    cache's order; the host tensors must be page-locked (pin_experts), which
    also makes them contiguous."""
    import codec
    from hostpool import to_tiles
    n = experts.num_experts
    pools = []
    lib = hipfetch.require()
    for host in (experts.w13_weight, experts.w2_weight):
        if not lib.is_page_locked(host):
            raise RuntimeError("CODED_POOL needs pinned expert tensors; run pin_experts first")
        raw = host.view(torch.uint8)
        rec = (to_tiles(raw) if experts._dc_tiles else raw).reshape(n, -1).numpy()
        pools.append(codec.CodedPool(rec, rec.shape[1], device))
    return tuple(pools)


def _copy_pairs(experts):
    """(host, cache) byte views moved on a miss (bin/devcache.py:170-181)."""
    return (
        (experts.w13_weight.view(torch.uint8).reshape(-1),
         experts._dc_w13.view(torch.uint8).reshape(-1)),
        (experts.w2_weight.view(torch.uint8).reshape(-1),
         experts._dc_w2.view(torch.uint8).reshape(-1)),
        (experts.w13_scale_inv.view(torch.uint8).reshape(-1),
         experts._dc_s13.view(torch.uint8).reshape(-1)),
        (experts.w2_scale_inv.view(torch.uint8).reshape(-1),
         experts._dc_s2.view(torch.uint8).reshape(-1)),
    )


def _device_ptr(lib, host: torch.Tensor) -> int:
    """Device address of a page-locked host tensor, cached by host address
    (bin/devcache.py:194,213-217)."""
    key = host.data_ptr()
    base = _dev_ptr_cache.get(key)
    if base is None:
        if not lib.is_page_locked(host):
            raise RuntimeError("expected a contiguous page-locked CPU tensor; run pin_experts "
                               "first (offload.pin_experts)")
        base = lib.device_ptr_of(key)
        _dev_ptr_cache[key] = base
    return base


def forget_host_memory(lo: int, hi: int) -> None:
    """Drop the cached device addresses of host buffers in [lo, hi), memory
    about to be freed: an address the allocator hands out again may then be
    pageable, and a stale entry would skip the page-locked check and send
    the fetch kernel to unmapped memory."""
    for k in [k for k in _dev_ptr_cache if lo <= k < hi]:
        del _dev_ptr_cache[k]


def _fetch_pairs(experts, lib):
    """[(src device address, dst address, bytes per record, tile_k)] for the
    4 buffers; tile_k is K of the w13/w2 matrices when the slots are tiled."""
    pairs = experts._dc_pairs
    if pairs is None:
        pairs = []
        ks = (experts.w13_weight.shape[-1], experts.w2_weight.shape[-1], 0, 0)
        for (host, cache), k in zip(_copy_pairs(experts), ks):
            per = host.numel() // experts.num_experts
            pairs.append((_device_ptr(lib, host), cache.data_ptr(), per,
                          k if experts._dc_tiles else 0))
        experts._dc_pairs = pairs
    return pairs


def _note_backend() -> None:
    global _BACKEND_NOTED
    if FETCH_BACKEND not in _BACKENDS:
        raise ValueError(f"FETCH_BACKEND must be one of {_BACKENDS}, got {FETCH_BACKEND!r}")
    if FETCH_BACKEND != "hip" and not _BACKEND_NOTED:
        _BACKEND_NOTED = True
        print(f"fetch backend {FETCH_BACKEND!r} maps to the HIP fetch kernel",
              file=_sys.stderr, flush=True)


def _call_ids(experts, topk_ids: torch.Tensor) -> torch.Tensor:
    """One decode call's ids, flat, int32 or int64, checked against the
    cache's capacity and the per-call scratch."""
    k = topk_ids.numel()
    if k > experts._dc_cap:
        # more ids than slots would make the table hand out a slot twice in
        # one call; the reference's gather path handles such calls
        raise ValueError(f"{k} ids exceed the cache capacity {experts._dc_cap}; "
                         "use offload.offloaded_forward for this call")
    if k > experts._dc_out.numel():
        raise ValueError(f"{k} ids exceed the preallocated scratch ({experts._dc_out.numel()})")
    ids = topk_ids.reshape(-1)
    return ids if ids.dtype in (torch.int32, torch.int64) else ids.to(torch.int32)


def _dev_resolve(experts, topk_ids: torch.Tensor, lib) -> torch.Tensor:
    """The slot resolve of dev_resolve_and_fetch alone: slots [k] int32 and
    the miss list in experts._dc_fexp/_dc_fslot/_dc_nmiss, no sync."""
    k = topk_ids.numel()
    ids = _call_ids(experts, topk_ids)
    lib.resolve_slots(ids, experts._dc_slot_of, experts._dc_slot_expert, experts._dc_stamp,
                      experts._dc_step, experts._dc_out, experts._dc_fslot, experts._dc_fexp,
                      experts._dc_nmiss, experts._dc_stats)
    return experts._dc_out[:k]


def dev_resolve_and_fetch(experts, topk_ids: torch.Tensor) -> torch.Tensor:
    """Resolve ids to slots, fetching misses.  Returns slot indices (int32),
    no sync (bin/devcache.py:230-255)."""
    _note_backend()
    lib = hipfetch.require()
    k = topk_ids.numel()
    _dev_resolve(experts, topk_ids, lib)
    coded = getattr(experts, "_dc_coded", None)
    if coded is None:
        lib.fetch(_fetch_pairs(experts, lib), experts._dc_fexp, experts._dc_fslot,
                  experts._dc_nmiss, max_jobs=k, blocks_per_job=CPP_BLOCKS_PER_JOB)
    else:
        # weights decoded from the coded pools, scales copied raw
        cap = experts._dc_cap
        for pool, cache in zip(coded, (experts._dc_w13, experts._dc_w2)):
            pool.fetch(cache.view(torch.uint8).reshape(cap, -1), experts._dc_fexp,
                       experts._dc_fslot, experts._dc_nmiss, max_jobs=k)
        lib.fetch(_fetch_pairs(experts, lib)[2:], experts._dc_fexp, experts._dc_fslot,
                  experts._dc_nmiss, max_jobs=k, blocks_per_job=CPP_BLOCKS_PER_JOB)
    return experts._dc_out[:k]


def dev_cached_forward(self, x, topk_ids, topk_weights):
    """MoEExperts.forward using the device-resident cache (bin/devcache.py:258-277).
    Decode calls (one row) only; every other call takes offload's gather, and
    so does a row with more ids than the cache has slots (the table would
    hand a slot to two of them)."""
    import offload
    cap = getattr(self, "_dc_cap", 0)
    if topk_ids.shape[0] != 1 or not cap or topk_ids.numel() > cap:
        return offload.offloaded_forward(self, x, topk_ids, topk_weights)
    k = topk_ids.numel()
    H = x.shape[-1]
    if (FUSED_FFN and self._dc_tiles and getattr(self, "_dc_coded", None) is None
            and H % 512 == 0 and k <= 16 and x.dtype == torch.bfloat16 and x.is_contiguous()
            and topk_weights.dtype in (torch.float32, torch.bfloat16)):
        # the resolve, the misses' fetch and every pick's gate/up in one
        # launch (its workgroups make the decisions of moe_resolve_slots
        # from the table), the down projection and the table's update in
        # the next
        _note_backend()
        lib = hipfetch.require()
        ids = _call_ids(self, topk_ids)
        inter = self._dc_w2.shape[-1]
        out = torch.empty_like(x)
        ws = torch.empty(k * inter * 4, dtype=torch.uint8, device=x.device)
        lib.resolve_fetch_ffn(ids, (self._dc_slot_of, self._dc_slot_expert, self._dc_stamp,
                                    self._dc_step), self._dc_next, self._dc_out, self._dc_fslot,
                              self._dc_fexp, self._dc_nmiss, _fetch_pairs(self, lib),
                              CPP_BLOCKS_PER_JOB, x, topk_weights.reshape(-1).contiguous(),
                              self._dc_w13, self._dc_s13, self._dc_w2, self._dc_s2, out, ws,
                              stats=self._dc_stats)
        return out
    slots = dev_resolve_and_fetch(self, topk_ids)
    return fp8_moe_forward(x, slots.reshape(topk_ids.shape), topk_weights, self._dc_w13,
                           self._dc_s13, self._dc_w2, self._dc_s2, layout=cache_layout(self))


def install_dev_cache(model, device, capacity: int) -> int:
    """Give every offloaded layer a device cache of `capacity` slots and
    route the experts class's forward through dev_cached_forward; returns how
    many layers got one (bin/devcache.py:280-301).  The fetch kernel reads
    host memory directly, so the expert buffers must be page-locked first
    (offload.pin_experts)."""
    from moe import MoEExperts
    n = 0
    classes = set()
    for layer in model.backbone.model.layers:
        experts = getattr(layer.mlp, "experts", None)
        if experts is None or experts.w13_weight.device.type != "cpu":
            continue
        if not hipfetch.require().is_page_locked(experts.w13_weight):
            raise RuntimeError("the expert buffers are pageable; the device cache fetches "
                               "from page-locked memory only (call offload.pin_experts)")
        init_dev_cache(experts, device, capacity)
        classes.add(type(experts))
        n += 1
    # the class the model's experts are built from (upstream's MoEExperts in
    # the reference's model); this package's stand-in when there are none
    for cls in classes or {MoEExperts}:
        if not hasattr(cls, "_stock_forward"):
            cls._stock_forward = cls.forward
        cls.forward = dev_cached_forward
    return n


def cache_stats(experts) -> tuple[int, int]:
    """(hits, misses) counted on the device since init (one host sync)."""
    s = experts._dc_stats.tolist()
    return int(s[0]), int(s[1])
