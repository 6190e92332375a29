"""Device-side prefill gather: the experts a multi-token call routes to are
gathered once and the grouped FP8 kernels run on them, with no host
synchronisation anywhere.

The reference's prefill (bin/offload.py:137-239) takes the distinct ids with
`torch.unique(topk_ids.cpu())` (a host sync per layer), reads the device
cache table back with `slot_of.cpu()` for the hybrid gather, copies each
expert with its own DMA and renumbers the ids on the host.  Here the same
steps are device launches whose sizes are read on the GPU:

    moe_permute         ids -> per-expert counts (and the stable token sort)
    moe_unique_inverse  counts -> distinct experts uniq[n] (ascending, as
                        torch.unique) and every pair renumbered into uniq
    moe_gather_plan     (hybrid only) uniq -> experts resident in the device
                        cache vs the rest; the table is only read
    moe_fetch           host records -> gather rows (and, hybrid, cache slots
                        -> gather rows, device to device), one launch each
    fp8_moe_forward     grouped W8A8 FFN on the gather buffers with the
                        renumbered ids (+ residual)

Expert storage is either the packed record pool (hostpool.HostPool, one
buffer) or the reference's four per-layer buffers w13/w2/s13/s2
(bin/devcache.py:170-181); `DevicePrefill` works on a list of buffers either
way.  A packed pool may also be held entropy-coded (codec.CodedPool); the
host part of the gather then decodes it into the same rows
(moe_fetch_coded).
"""
from __future__ import annotations

import torch

import hipfetch
from hostpool import DRAMA3, RecordLayout

# Fetch workgroups per job: the host link saturates at 3 (~192 KiB in
# flight); device-to-device copies from the cache want many more.
HOST_BLOCKS_PER_JOB = 3
CACHE_BLOCKS_PER_JOB = 64


class DevicePrefill:
    """Scratch and launches for one multi-token expert call at a time.

    gather:  device buffers [n_experts, ...] the experts are gathered into,
             one per storage buffer (packed: one uint8 [n, record]; the
             reference's layout: w13, w2, s13, s2)
    views:   (w13, s13, w2, s2) over the gather buffers, as fp8_moe_forward
             takes them
    layout:  byte order of the gathered w13/w2 (hipfetch.LAYOUT_*)
    tile_k:  per gather buffer, the fetch's tile_k for copies from the host
             (K of a row-major host matrix written in tile order; 0 copies
             bytes).  Copies between device buffers always copy bytes."""

    def __init__(self, gather: list[torch.Tensor], views, top_k: int, max_tokens: int,
                 hidden: int, inter: int, layout: int = hipfetch.LAYOUT_ROWS,
                 tile_k: list[int] | None = None):
        self.lib = hipfetch.require()
        self.gather = gather
        self.views = views
        self.layout = layout
        self.tile_k = list(tile_k) if tile_k is not None else [0] * len(gather)
        self.E = gather[0].shape[0]
        self.K, self.max_tokens = top_k, max_tokens
        self.dev = gather[0].device
        self.row_bytes = [g[0].numel() * g.element_size() for g in gather]
        P = max_tokens * top_k
        i32 = dict(dtype=torch.int32, device=self.dev)
        E = self.E
        self.counts = torch.zeros(E, **i32)
        self.offsets = torch.zeros(E + 1, **i32)
        self.sorted = torch.zeros(P, **i32)
        self.pos = torch.zeros(P, **i32)
        self.n_unique = torch.zeros(1, **i32)
        self.uniq = torch.zeros(E, **i32)
        self.rank_of = torch.zeros(E, **i32)
        self.inverse = torch.zeros(P, **i32)
        self.rows = torch.arange(E, **i32)
        self.host_expert = torch.zeros(E, **i32)
        self.host_dst = torch.zeros(E, **i32)
        self.n_host = torch.zeros(1, **i32)
        self.cache_src = torch.zeros(E, **i32)
        self.cache_dst = torch.zeros(E, **i32)
        self.n_cache = torch.zeros(1, **i32)
        # {experts copied from the cache, experts fetched from the host}
        self.stats = torch.zeros(2, dtype=torch.int64, device=self.dev)
        self.ws = torch.empty(self.lib.fp8_moe_workspace(max_tokens, top_k, E, hidden, inter),
                              dtype=torch.uint8, device=self.dev)

    @classmethod
    def for_records(cls, n_experts: int, top_k: int, max_tokens: int, device,
                    layout: RecordLayout = DRAMA3) -> "DevicePrefill":
        """Gather buffer of packed records (805 MB at Drama-3 shapes)."""
        g = torch.empty((n_experts, layout.record_bytes), dtype=torch.uint8, device=device)
        return cls([g], layout.views(g), top_k, max_tokens, layout.hidden, layout.inter,
                   layout.code)

    @classmethod
    def for_experts(cls, experts, top_k: int, max_tokens: int, device,
                    tiles: bool = False, rows: list[torch.Tensor] | None = None
                    ) -> "DevicePrefill":
        """Gather buffers shaped like an experts module's four host buffers.
        tiles: the host's row-major w13/w2 land in MFMA tile order, which the
        FFN then reads as LAYOUT_TILES (the scales are copied as they are).
        rows: another DevicePrefill's gather buffers to share (its calls and
        this one's must be ordered on one stream); new ones by default."""
        names = ("w13_weight", "w2_weight", "w13_scale_inv", "w2_scale_inv")
        if rows is None:
            bufs = [torch.empty_like(getattr(experts, n), device=device) for n in names]
        else:
            bufs = list(rows)
            for b, n in zip(bufs, names):
                h = getattr(experts, n)
                if b.shape != h.shape or b.dtype != h.dtype:
                    raise ValueError(f"shared gather rows do not match {n}")
        views = (bufs[0], bufs[2], bufs[1], bufs[3])
        hidden, inter = experts.w13_weight.shape[2], experts.w2_weight.shape[2]
        if tiles:
            return cls(bufs, views, top_k, max_tokens, hidden, inter, hipfetch.LAYOUT_TILES,
                       [hidden, inter, 0, 0])
        return cls(bufs, views, top_k, max_tokens, hidden, inter)

    def gather_experts(self, ids: torch.Tensor, host_src: list[int] | None, cache=None,
                       coded=None) -> torch.Tensor:
        """Distinct experts of ids [T, K] into the gather rows (row i holds
        expert uniq[i]); returns the renumbered ids [T, K] int32 (a view of
        this object's scratch).

        host_src: device addresses of the page-locked host buffers, one per
        gather buffer.  cache: None, or (slot_of, cap, [cache buffer
        addresses, one per gather buffer]) to serve resident experts from the
        device cache (hybrid gather; the table is only read).  coded: a
        codec.CodedPool of the layer's records, read instead of host_src
        (packed records only)."""
        T, K = ids.shape
        if T > self.max_tokens or K != self.K:
            raise ValueError(f"call of {T}x{K} ids exceeds the prefill scratch "
                             f"({self.max_tokens}x{self.K})")
        if coded is not None:
            if len(self.gather) != 1 or self.row_bytes[0] != coded.record_bytes:
                raise ValueError("a coded pool serves a gather buffer of packed records")
        elif host_src is None or len(host_src) != len(self.gather):
            raise ValueError("one host buffer per gather buffer")
        P = T * K
        lib = self.lib
        lib.permute(ids, self.E, self.counts, self.offsets, self.sorted[:P], self.pos[:P])
        lib.unique_inverse(ids, self.E, self.counts, self.n_unique, self.uniq, self.rank_of,
                           self.inverse[:P])
        dst = [g.data_ptr() for g in self.gather]

        def from_host(experts, rows, n):
            if coded is not None:
                coded.fetch(self.gather[0], experts, rows, n, max_jobs=self.E)
            else:
                pairs = list(zip(host_src, dst, self.row_bytes, self.tile_k))
                lib.fetch(pairs, experts, rows, n, max_jobs=self.E,
                          blocks_per_job=HOST_BLOCKS_PER_JOB)

        if cache is None:
            # no cache: the plan sends every expert to the host list (and
            # counts them in self.stats)
            lib.gather_plan(self.uniq, self.n_unique, None, 0, self.host_expert,
                            self.host_dst, self.n_host, self.cache_src, self.cache_dst,
                            self.n_cache, self.stats)
        else:
            slot_of, cap, cache_src = cache
            if len(cache_src) != len(self.gather):
                raise ValueError("one cache buffer per gather buffer")
            lib.gather_plan(self.uniq, self.n_unique, slot_of, cap, self.host_expert,
                            self.host_dst, self.n_host, self.cache_src, self.cache_dst,
                            self.n_cache, self.stats)
            cache_pairs = [(s, d, b) for s, d, b in zip(cache_src, dst, self.row_bytes)]
            lib.fetch(cache_pairs, self.cache_src, self.cache_dst, self.n_cache,
                      max_jobs=self.E, blocks_per_job=CACHE_BLOCKS_PER_JOB)
        from_host(self.host_expert, self.host_dst, self.n_host)
        return self.inverse[:P].view(T, K)

    def forward(self, x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
                host_src: list[int] | None, cache=None, out: torch.Tensor | None = None,
                residual: torch.Tensor | None = None, coded=None) -> torch.Tensor:
        """MoE output [T, H] bf16 for x [T, H] with the experts read from the
        host buffers, or the coded pool (and, hybrid, the device cache)."""
        local = self.gather_experts(ids, host_src, cache, coded)
        if out is None:
            out = torch.empty_like(x)
        w13, s13, w2, s2 = self.views
        self.lib.fp8_moe_forward(x, local, weights, w13, s13, w2, s2, out, self.ws, mode=2,
                                 residual=residual, layout=self.layout)
        return out

    def copy_stats(self) -> tuple[int, int]:
        """(experts copied from the device cache, fetched from the host) since
        construction (one host sync)."""
        s = self.stats.tolist()
        return int(s[0]), int(s[1])
