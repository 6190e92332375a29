"""The 40-layer batch-1 decode step with experts offloaded, captured in one
hipGraph.

Per layer, all on one stream, nothing synchronising and nothing allocating:

    h     = x W_stub[l]^T                     non-expert compute (bf16 matmul stub)
    ids,w = router(h, gate[l], bias[l])       top-8 of 256 (HIP)
    slots = resolve(ids, table[l])            device LRU, misses queued (HIP)
    fetch(pool[l] -> cache[l], misses)        zero-copy host -> HBM (HIP)
    y     = fp8_moe_forward(h, slots, w)      W8A8 expert FFN on the cache (HIP)
    x     = h + y

The router, resolve, fetch and expert FFN are three launches
(moe_route_fetch_ffn: the logits; the route, the misses' fetch and the gate/up
half of the FFN, every workgroup resolving the call itself from a
double-buffered slot table, the workgroups that fetch a miss's rows running
its gate/up MFMAs on them as they arrive; the down half).  With
fused_ffn=False the FFN is its own two launches after moe_route_fetch's two;
with fused_fetch=False the route is moe_route_resolve and the fetch a launch
of its own.  With coded pools the route and the decode of the misses share
a launch (moe_route_fetch_coded) and the FFN is its own two.

With `shared_expert`, the step is the full MoE block, one call after the
fetch: the gated bf16 shared expert rides in the two routed GEMV launches
(moe_fp8_moe_block_forward), which also add the residual,

    x = h + (y + sigmoid(h w_sg) * shared(h))

and after the last layer a device flag records whether x is finite (the
decode graph's finiteness guard).

This is the path Drama3DecodeGraphs captures around dev_cached_forward in the
reference (bin/prefix_kv.py:383-457 driving bin/devcache.py:258-277), with
the rest of the transformer replaced by one [2048, 2048] matmul per layer.
Expert popularity follows a per-layer Zipf law that is redrawn every
`drift_every` steps, injected as a router bias (log-popularity + Gumbel
noise); the bias for the next step is staged into a fixed buffer before each
replay.

mode "cached": per-layer cache of `capacity` packed records, LRU on device.
mode "nocache": every routed expert is fetched on every step (0 % hit; the
reference's uncached per-expert transfer), into 8 fixed slots: the router,
the fetch and the gate/up in one launch as on the cached path
(moe_route_fetch_ffn_uncached), or with fused_fetch off, moe_router_topk +
moe_fetch + moe_fp8_moe_forward.

With `coded_pool`, each layer's records are also held entropy-coded in host
memory (codec.CodedPool) and the fetch decodes them into the same cache
slots (moe_fetch_coded): the same bytes land in HBM, fewer cross the link.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

import hipfetch
import synth
from hostpool import DRAMA3, HostPool, RecordLayout


def stub_linear(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor, x_add=None) -> None:
    """The non-expert stand-in, out = x w^T with w [out, in] bf16 (an
    nn.Linear without bias); with x_add, out = (x + x_add) w^T, the bf16
    add folded into the product's loads.  moe_linear_bf16 takes up to 4
    tokens on the vector units, one pass over the weights (3.55 us for
    2048 x 2048 at one token on MI355X, against 6.9 us for torch.mv and
    12.0 us for a 1-row torch.mm), and 5 to 128 on the matrix cores (5.3 /
    7.7 / 11.2 us at 8 / 32 / 128 tokens, against 10.9 / 11.1 / 11.2 for
    torch.mm); beyond that, or for shapes it does not take, a torch
    matrix product."""
    T, K = x.shape
    if T <= 4 or (T <= 128 and x_add is None and K % 64 == 0 and w.shape[0] % 16 == 0):
        hipfetch.require().linear_bf16(x, w, out, x_add=x_add)
    else:
        torch.mm(x if x_add is None else x + x_add, w.t(), out=out)


@dataclass
class DecodeConfig:
    layers: int = 40
    n_experts: int = 256
    top_k: int = 8
    hidden: int = 2048
    inter: int = 512
    capacity: int = 96
    mode: str = "cached"            # "cached" | "nocache"
    seed: int = 0
    schedule_steps: int = 200
    drift_every: int = 50
    zipf_s: float = 1.1
    gate_std: float = 0.002
    blocks_per_job: int = 3
    fused_fetch: bool = True        # router + resolve + fetch in two launches (moe_route_fetch)
    fused_ffn: bool = True          # ... and the FFN's gate/up in the same launch (moe_route_fetch_ffn)
    # fetch workgroups per miss on that path (MI355X, ms per step): 7.712 /
    # 7.700 / 7.880 / 7.990 at 3 / 4 / 5 / 6 when the plain pieces were
    # dealt round robin (62 % hit); with them dealt by counter and the first
    # piece read early, 7.798 / 7.757 / 7.743 / 7.773 (100-step windows,
    # alternating), and 7.786 / 7.767 at 4 / 5 over six 200-step windows
    ffn_blocks_per_job: int = 5
    noncoherent_pool: bool = False
    shared_expert: bool = False     # the MoE block's gated bf16 shared expert
    shared_inter: int = 512
    coded_pool: bool = False        # fetch from entropy-coded host records
    coded_workgroups: int = 32
    router_logits: str = "bf16"     # the gate's output dtype: "bf16" (a bf16 Linear) or "f32"


def fill_pool_on_gpu(pool: HostPool, seed: int, layer: int, device, chunk: int = 64,
                     std: float = 0.02) -> None:
    """Seeded N(0, std) weights, 128x128-block quantised, generated on the GPU
    and written into the page-locked pool as packed records."""
    lay = pool.layout
    H, I = lay.hidden, lay.inter
    g = torch.Generator(device=device).manual_seed(seed * 7919 + layer)
    for e0 in range(0, pool.n, chunk):
        n = min(chunk, pool.n - e0)
        w13, s13 = synth.quantize_blocks(torch.randn((n, 2 * I, H), generator=g, device=device) * std)
        w2, s2 = synth.quantize_blocks(torch.randn((n, H, I), generator=g, device=device) * std)
        pool.write(e0, lay.pack(w13, s13, w2, s2))
    torch.cuda.synchronize(device)


def resident_table(n_experts: int, device):
    """A double-buffered slot table over records that are all resident
    (slot e holds expert e, both buffers; stamps -E..-1): given to
    moe_route_fetch_ffn with the records as the cache, every pick hits, no
    miss is queued and the pool is never read, so the launch is the route
    and the gate/up of the all-resident decode step."""
    i32 = dict(dtype=torch.int32, device=device)
    ar = torch.arange(n_experts, **i32)
    slot_of = ar.repeat(2, 1).contiguous()
    slot_expert = ar.repeat(2, 1).contiguous()
    stamp = (torch.arange(n_experts, dtype=torch.int64, device=device) - n_experts).repeat(2, 1)
    step = torch.zeros(1, dtype=torch.int64, device=device)
    return slot_of, slot_expert, stamp.contiguous(), step


class DecodeHarness:
    def __init__(self, cfg: DecodeConfig, device=None, pools: list[HostPool] | None = None,
                 coded: list | None = None):
        self.cfg = cfg
        self.lib = hipfetch.require()
        self.dev = torch.device(device or "cuda:0")
        self.layout = pools[0].layout if pools else RecordLayout(cfg.hidden, cfg.inter)
        if (self.layout.hidden, self.layout.inter) != (cfg.hidden, cfg.inter):
            raise ValueError("the pools' record layout does not match the config's shapes")
        L, E, K, H = cfg.layers, cfg.n_experts, cfg.top_k, cfg.hidden
        dev = self.dev
        if pools is None:
            pools = []
            for l in range(L):
                p = HostPool(E, self.layout, noncoherent=cfg.noncoherent_pool)
                fill_pool_on_gpu(p, cfg.seed, l, dev)
                pools.append(p)
        self.pools = pools
        C = cfg.capacity if cfg.mode == "cached" else K
        if C < K:
            raise ValueError(f"capacity {C} < top_k {K}")
        self.C = C
        RB = self.layout.record_bytes
        self.cache = [torch.zeros((C, RB), dtype=torch.uint8, device=dev) for _ in range(L)]
        self.views = [self.layout.views(c) for c in self.cache]
        # slot tables and per-layer scratch
        i32 = dict(dtype=torch.int32, device=dev)
        # double-buffered slot tables (moe_route_fetch; buffer 0 only otherwise)
        self.tab_slot_of = torch.empty((L, 2, E), **i32)
        self.tab_slot_expert = torch.empty((L, 2, C), **i32)
        self.tab_stamp = torch.empty((L, 2, C), dtype=torch.int64, device=dev)
        self.step = [torch.empty(1, dtype=torch.int64, device=dev) for _ in range(L)]
        self.stats = torch.zeros((L, 2), dtype=torch.int64, device=dev)
        self.ids = torch.zeros((L, 1, K), **i32)
        self.wts = torch.zeros((L, 1, K), dtype=torch.float32, device=dev)
        self.logits = torch.zeros((L, 1, E), dtype=torch.float32, device=dev)
        self.out_slot = torch.zeros((L, 1, K), **i32)
        self.fslot = torch.zeros((L, K), **i32)
        self.fexp = torch.zeros((L, K), **i32)
        self.nmiss = torch.zeros((L, 1), **i32)
        self.fixed_slots = torch.arange(K, **i32).view(1, K)
        self.all_miss = torch.full((1,), K, **i32)
        self.reset_tables()
        # non-expert stub, router gates, routing schedule
        g = torch.Generator(device=dev).manual_seed(cfg.seed + 1)
        # std 1/sqrt(H) keeps the residual stream's scale from layer to layer;
        # [out, in] per layer, the layout of an nn.Linear weight
        self.w_stub = (torch.randn((L, H, H), generator=g, device=dev) * (1.0 / H ** 0.5)).to(torch.bfloat16)
        self.gate = (torch.randn((L, E, H), generator=g, device=dev) * cfg.gate_std).to(torch.bfloat16)
        rng = np.random.default_rng(cfg.seed)
        bias = synth.decode_route_bias(rng, cfg.schedule_steps, L, E, cfg.zipf_s, cfg.drift_every)
        self.bias_all = torch.from_numpy(bias).to(dev)
        self.bias_live = torch.empty((L, E), dtype=torch.float32, device=dev)
        self.x0 = synth.hidden_states(cfg.seed, 1, H, device="cpu").to(dev)
        self.x = self.x0.clone()
        self.h = torch.empty((1, H), dtype=torch.bfloat16, device=dev)
        self.y = torch.empty((1, H), dtype=torch.bfloat16, device=dev)
        ws = self.lib.fp8_moe_workspace(1, K, C, H, cfg.inter)
        self.ws = torch.empty(ws, dtype=torch.uint8, device=dev)
        self.pairs = [p.fetch_pair(c) for p, c in zip(self.pools, self.cache)]
        self.coded = None
        if cfg.coded_pool:
            if coded is None:
                coded = build_coded_pools(self.pools, self.layout, dev)
            if len(coded) != L:
                raise ValueError(f"{len(coded)} coded pools for {L} layers")
            self.coded = coded
        # the step takes moe_route_fetch (router + resolve + fetch; for coded
        # pools moe_route_fetch_coded), decided once
        self.fused = cfg.mode == "cached" and cfg.fused_fetch
        # ... and the FFN with it (raw packed tile-ordered records)
        self.fused_ffn = (self.fused and self.coded is None and cfg.fused_ffn and
                          self.layout.tiled and cfg.hidden % 512 == 0 and cfg.top_k <= 16)
        # at 0 % hit: the same three launches with no slot table
        # (moe_route_fetch_ffn_uncached), every pick fetched into slot k; no
        # hit/miss counts at 0 % hit, as on the separate launches
        self.fused_uncached = (cfg.mode == "nocache" and cfg.fused_fetch and cfg.fused_ffn and
                               self.coded is None and self.layout.tiled and
                               cfg.hidden % 512 == 0 and cfg.top_k <= 16)
        if cfg.shared_expert:
            # seeded bf16 shared experts, resident (6 MiB per layer at 2048 x 512)
            g2 = torch.Generator(device=dev).manual_seed(cfg.seed + 3)
            Is = cfg.shared_inter
            rnd = lambda *s, std: (torch.randn(s, generator=g2, device=dev) * std).to(torch.bfloat16)
            # N(0, 0.02) like the routed experts, down N(0, 0.005): with no norm in
            # the stub, a second quadratic term per layer at the routed experts'
            # scale grows the residual stream past bf16 range within 40 layers
            self.sh_wg = rnd(L, Is, H, std=0.02)
            self.sh_wu = rnd(L, Is, H, std=0.02)
            self.sh_wd = rnd(L, H, Is, std=0.005)
            self.sh_wsg = rnd(L, H, std=0.02)
            self.ws_block = torch.empty(
                self.lib.fp8_moe_block_workspace(1, K, C, H, cfg.inter, Is), dtype=torch.uint8,
                device=dev)
        self.finite = torch.ones(1, dtype=torch.int32, device=dev)
        self.graph = None
        self.cursor = 0

    def _tables(self) -> tuple[list, list, list]:
        """Each layer's current slot table (slot_of, slot_expert, stamp views;
        one host sync): buffer step & 1 on the fused path, else buffer 0."""
        L = self.cfg.layers
        if self.fused:
            buf = (torch.cat(self.step).cpu() & 1).tolist()
        else:
            buf = [0] * L
        return ([self.tab_slot_of[l, b] for l, b in zip(range(L), buf)],
                [self.tab_slot_expert[l, b] for l, b in zip(range(L), buf)],
                [self.tab_stamp[l, b] for l, b in zip(range(L), buf)])

    @property
    def slot_of(self) -> list:
        return self._tables()[0]

    @property
    def slot_expert(self) -> list:
        return self._tables()[1]

    @property
    def stamp(self) -> list:
        return self._tables()[2]

    def shared(self, l: int):
        """Layer l's shared expert (gate, up, down, sigmoid gate)."""
        return self.sh_wg[l], self.sh_wu[l], self.sh_wd[l], self.sh_wsg[l]

    # -------------------------------------------------------------- state
    def reset_tables(self) -> None:
        for l in range(self.cfg.layers):
            self.lib.slots_init(self.tab_slot_of[l, 0], self.tab_slot_expert[l, 0],
                                self.tab_stamp[l, 0], self.step[l])
        self.stats.zero_()

    def stage(self, s: int) -> None:
        """Bias of schedule step s into the fixed buffer the graph reads."""
        self.bias_live.copy_(self.bias_all[s % self.cfg.schedule_steps])

    # -------------------------------------------------------------- step
    def layer(self, l: int) -> None:
        cfg, lib = self.cfg, self.lib
        stub_linear(self.x, self.w_stub[l], self.h)
        w13, s13, w2, s2 = self.views[l]
        if self.fused_ffn:
            # the whole layer's MoE (block) in three launches; x = h + MoE(h)
            lib.route_fetch_ffn(self.h, self.gate[l], self.bias_live[l], cfg.top_k,
                                self.logits[l], self.ids[l], self.wts[l], self.tab_slot_of[l],
                                self.tab_slot_expert[l], self.tab_stamp[l], self.step[l],
                                self.out_slot[l], self.fslot[l], self.fexp[l], self.nmiss[l],
                                self.pools[l].dev_ptr, self.cache[l], cfg.inter,
                                cfg.ffn_blocks_per_job, self.x,
                                self.ws_block if cfg.shared_expert else self.ws,
                                residual=self.h, stats=self.stats[l],
                                logit_dtype=cfg.router_logits,
                                shared=self.shared(l) if cfg.shared_expert else None)
            return
        if self.fused_uncached:
            lib.route_fetch_ffn_uncached(self.h, self.gate[l], self.bias_live[l], cfg.top_k,
                                         self.logits[l], self.ids[l], self.wts[l],
                                         self.out_slot[l], self.fslot[l], self.fexp[l],
                                         self.nmiss[l], self.pools[l].dev_ptr, self.cache[l],
                                         cfg.inter, cfg.ffn_blocks_per_job, self.x,
                                         self.ws_block if cfg.shared_expert else self.ws,
                                         residual=self.h, logit_dtype=cfg.router_logits,
                                         shared=self.shared(l) if cfg.shared_expert else None)
            return
        if self.fused and self.coded is not None:
            # router, then resolve + decode of the misses' coded records
            c = self.coded[l]
            lib.route_fetch_coded(self.h, self.gate[l], self.bias_live[l], cfg.top_k,
                                  self.logits[l], self.ids[l], self.wts[l], self.tab_slot_of[l],
                                  self.tab_slot_expert[l], self.tab_stamp[l], self.step[l],
                                  self.out_slot[l], self.fslot[l], self.fexp[l], self.nmiss[l],
                                  c.dev_ptr, c.rec_off, c.blk_off, c.record_bytes, c.fp8_bytes,
                                  c.lut, self.cache[l], workgroups=cfg.coded_workgroups,
                                  stats=self.stats[l], logit_dtype=cfg.router_logits)
            slots = self.out_slot[l]
        elif self.fused:
            # router, then resolve + miss fetch in one launch (double-buffered table)
            lib.route_fetch(self.h, self.gate[l], self.bias_live[l], cfg.top_k, self.logits[l],
                            self.ids[l], self.wts[l], self.tab_slot_of[l],
                            self.tab_slot_expert[l], self.tab_stamp[l], self.step[l],
                            self.out_slot[l], self.fslot[l], self.fexp[l], self.nmiss[l],
                            [self.pairs[l]], cfg.blocks_per_job, stats=self.stats[l],
                            logit_dtype=cfg.router_logits)
            slots = self.out_slot[l]
        elif cfg.mode == "cached":
            # router + slot resolve (two launches), then the miss fetch
            lib.route_resolve(self.h, self.gate[l], self.bias_live[l], cfg.top_k, self.logits[l],
                              self.ids[l], self.wts[l], self.tab_slot_of[l, 0],
                              self.tab_slot_expert[l, 0], self.tab_stamp[l, 0], self.step[l],
                              self.out_slot[l], self.fslot[l], self.fexp[l], self.nmiss[l],
                              self.stats[l], logit_dtype=cfg.router_logits)
            self.fetch(l, self.fexp[l], self.fslot[l], self.nmiss[l])
            slots = self.out_slot[l]
        else:
            lib.router_topk(self.h, self.gate[l], self.bias_live[l], cfg.top_k, self.logits[l],
                            self.ids[l], self.wts[l], logit_dtype=cfg.router_logits)
            self.fetch(l, self.ids[l].view(-1), self.fixed_slots.view(-1), self.all_miss)
            slots = self.fixed_slots
        if cfg.shared_expert:
            # x = h + (routed + shared): the whole block in the two decode launches
            lib.fp8_moe_block_forward(self.h, slots, self.wts[l], w13, s13, w2, s2,
                                      self.shared(l), self.x, self.ws_block, residual=self.h,
                                      layout=self.layout.code)
        else:
            # x = h + MoE(h), the residual add fused into the down kernel
            lib.fp8_moe_forward(self.h, slots, self.wts[l], w13, s13, w2, s2, self.x, self.ws,
                                residual=self.h, layout=self.layout.code)

    def fetch(self, l: int, experts, slots, nmiss) -> None:
        """Layer l's miss fetch: records experts[j] into cache slots slots[j],
        j < nmiss[0], raw or entropy-coded."""
        cfg = self.cfg
        if self.coded is not None:
            self.coded[l].fetch(self.cache[l], experts, slots, nmiss, max_jobs=cfg.top_k,
                                workgroups=cfg.coded_workgroups)
        else:
            self.lib.fetch([self.pairs[l]], experts, slots, nmiss, max_jobs=cfg.top_k,
                           blocks_per_job=cfg.blocks_per_job)

    def step_eager(self) -> None:
        # every step starts from the same input token state (the stub has no
        # embedding); feeding the last layer's output back would compound
        # the residual stream's growth over thousands of layer applications
        self.x.copy_(self.x0)
        for l in range(self.cfg.layers):
            self.layer(l)
        if self.cfg.shared_expert:
            self.lib.all_finite(self.x, self.finite)

    def capture(self) -> torch.cuda.CUDAGraph:
        s = torch.cuda.Stream(device=self.dev)
        s.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(s):
            self.stage(0)
            self.step_eager()                       # warm-up outside capture
        torch.cuda.current_stream(self.dev).wait_stream(s)
        torch.cuda.synchronize(self.dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step_eager()
        self.graph = g
        self.restart()
        return g

    def restart(self) -> None:
        """Empty caches, first input, schedule from step 0."""
        self.reset_tables()
        self.x.copy_(self.x0)
        self.cursor = 0
        torch.cuda.synchronize(self.dev)

    def replay(self, n: int = 1) -> None:
        for _ in range(n):
            self.stage(self.cursor)
            self.graph.replay()
            self.cursor += 1

    def hit_rate(self) -> tuple[int, int]:
        s = self.stats.sum(0).tolist()
        return int(s[0]), int(s[1])

    def close(self) -> None:
        self.graph = None
        for p in self.pools:
            p.close()
        self.pools = []
        for c in self.coded or []:
            c.close()
        self.coded = None


def build_coded_pools(pools: list[HostPool], layout: RecordLayout, device, threads: int = 16):
    """One CodedPool per layer from the raw pools (each coded with its own
    layer's code lengths), sharing one encode scratch buffer."""
    import codec
    need = hipfetch.require().codec_bound(layout.record_bytes, layout.off_s13) * max(p.n for p in pools)
    scratch = np.empty(need, dtype=np.uint8)
    return [codec.CodedPool(p.array, layout, device, threads=threads, scratch=scratch)
            for p in pools]
