// The decode step's MoE layer of one token from packed records in three
// launches: the router's logits; the route (top-k + slot resolve), the
// misses' fetch and the gate/up half of the expert FFN in one launch; the
// down half.  The separate form is moe_route_fetch followed by
// moe_fp8_moe_forward_ex (four launches); both give the same bytes.  The
// drop-in's form (fetch_gateup_kernel below) does the same on the
// reference's four buffers and single-buffer slot table, after a resolve
// launch (moe_fetch_ffn) or making the resolve itself (moe_resolve_fetch_ffn).
//
// Records: w13 [2I, H] | w2 [H, I] in MFMA tile order | s13 [2I/128, H/128]
// | s2 [H/128, I/128] f32, record_bytes apart in the host pool and in the
// cache.  In tile order the 16 rows 16g..16g+15 of w13 are 16H contiguous
// bytes, 2 KiB per 128-column K-block, each K-block holding the MFMA A
// operands of a wave: lane 16q + r finds row r, columns 32q..32q+15 at
// byte 16 * lane and columns 32q+16..32q+31 at 1024 + 16 * lane.
//
// The route + fetch + gate/up launch has two kinds of workgroups (128
// threads each); all of them first make the route on their first wave
// (route.hpp: the same decisions in every workgroup, workgroup 0 writing
// the outputs and the next table buffer) while the second wave quantises x
// into LDS.
//   * fetch workgroups (the first nfetch): the misses' records, cut into
//     units of 16 intermediate columns (the 16 gate rows and the 16 up rows
//     of those columns, 2 * H/512 pieces of 8 KiB) and plain 4 KiB pieces
//     (w2, the scales).  A unit's pieces go through one workgroup, which
//     stores them to the cache slot as they arrive and runs the gate/up
//     MFMAs on the bytes in its registers: the unit ends with the 16
//     SiLU(gate) * up values of the miss's pick.  Units go round robin over
//     the workgroups; then each wave takes plain pieces from a counter
//     until none is left, so the workgroups that receive host bytes sooner
//     move more of them.
//   * hit workgroups (top_k * I/16 of them, one per pick and unit): a hit's
//     16 gate rows (first wave) and 16 up rows (second wave) from its cache
//     slot; a pick that missed leaves its workgroup idle.
//   * with the MoE block's shared expert, workgroups for its gate/up rows
//     and sigmoid gate (the gate/up GEMV kernel's shared workgroups, the
//     same arithmetic); they need no route.  Its down rows then ride in the
//     down launch, which adds residual + (routed + sigmoid-gated shared).
// Every row sum is the in-order chain over its K-blocks of fma(block
// product, weight scale * x scale, sum) that the gate/up GEMV kernel forms,
// so the activations, and the down launch's output, are bit-identical to
// the separate launches'.  The fetch's link time hides the hits' gate/up,
// and the gate/up launch after the fetch goes away.
#include <hip/hip_ext.h>

#include "common.hpp"
#include "fetch.hpp"
#include "gemv.hpp"
#include "resolve.hpp"
#include "route.hpp"
#include "shared.hpp"

namespace moe {

constexpr int kStepThreads = 128;
constexpr int kPieceBytes = 8192;          // 128 threads x 4 x 16 bytes
constexpr int kHitChunk = 16;              // K-blocks of a hit tile in flight per lane

struct StepGeom {
  const char* pool;        // device address of host record 0
  char* cache;             // cache slot 0
  int64_t rb;              // record bytes (pool and cache stride)
  int64_t w13_bytes;       // 2 I H
  int64_t off_s13;         // w13_bytes + H I
  int32_t hidden, inter;
  int32_t gb;              // K-blocks per row: H / 128
  int32_t kq;              // pieces per 16-row group: H / 512
  int32_t units;           // units per record: I / 16
  int32_t plain;           // 4 KiB pieces from w13_bytes to the record's end
  int32_t nfetch;          // fetch workgroups (the first of the grid)
  int32_t* ticket;         // the plain pieces' counter, zeroed by the logits launch
};

__device__ __forceinline__ int32_t uniform(int32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// UNCACHED (moe_route_fetch_ffn_uncached): no slot table; every pick is a
// miss fetched into slot k (its place in the top-k), so the grid has no hit
// workgroups and the table arguments are unused.
template <bool UNCACHED, int PER, int PERC>
__global__ __launch_bounds__(kStepThreads) void route_fetch_gateup_kernel(
    StepGeom g, const uint16_t* __restrict__ x, const float* __restrict__ logits,
    int32_t n_experts, int32_t top_k, int32_t* __restrict__ ids, float* __restrict__ weights,
    int32_t* __restrict__ slot_of, int32_t* __restrict__ slot_expert,
    int64_t* __restrict__ stamp, int32_t cap, const int64_t* __restrict__ step_ptr,
    int32_t* __restrict__ out_slot, int32_t* __restrict__ fetch_slot,
    int32_t* __restrict__ fetch_expert, int32_t* __restrict__ nmiss_ptr,
    int64_t* __restrict__ stats, float* __restrict__ act, SharedRefs sh) {
  const int first_shared = g.nfetch + (UNCACHED ? 0 : top_k * g.units);
  if (static_cast<int>(blockIdx.x) >= first_shared) {
    // shared expert rows j0, j0 + 1 of this wave (gate and up each; row Is
    // is the sigmoid gate), the token's x; no barrier on this branch
    const int wv = threadIdx.x >> 6;
    const int ln = threadIdx.x & 63;
    const int j0 = ((static_cast<int>(blockIdx.x) - first_shared) * 2 + wv) * kSharedJPW;
    if (j0 > sh.inter) return;
    const uint16_t* rows[2 * kSharedJPW];
#pragma unroll
    for (int i = 0; i < kSharedJPW; ++i) {
      const int j = min(j0 + i, sh.inter);
      const bool gate_row = j == sh.inter;
      rows[2 * i] = gate_row ? sh.wsg : sh.wg + static_cast<int64_t>(j) * g.hidden;
      rows[2 * i + 1] = gate_row ? sh.wsg : sh.wu + static_cast<int64_t>(j) * g.hidden;
    }
    float sacc[2 * kSharedJPW][1];
    rows_dot_bf16<2 * kSharedJPW, 1, 4>(rows, x, g.hidden, 0, 1, g.hidden >> 3, ln, sacc);
    if (ln == 0) {
#pragma unroll
      for (int i = 0; i < kSharedJPW; ++i) {
        const int j = j0 + i;
        if (j < sh.inter) sh.act[j] = shared_act(sacc[2 * i][0], sacc[2 * i + 1][0]);
        else if (j == sh.inter) *sh.sig = shared_sig(sacc[2 * i][0]);
      }
    }
    return;
  }
  __shared__ __align__(16) uint8_t xq[kGemvMaxHidden];
  __shared__ float xs[kGemvMaxHidden / 128];
  __shared__ __align__(16) float dpart[2][kGemvMaxHidden / 128][16];
  __shared__ __align__(16) float upsum[16];
  __shared__ float swl[2][64];              // a unit's block scales, per wave
  __shared__ int32_t job_e[kMaxTopK], job_s[kMaxTopK], job_k[kMaxTopK], job_n;
  __shared__ int32_t pick_slot[kMaxTopK];   // a hit's slot, -1 for a miss
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4;
  // A fetch workgroup whose first unit is of job 0 (b < units) reads that
  // unit's first piece as soon as each wave knows the first miss (before
  // the resolve, which only decides where it is stored): its host reads
  // overlap the resolve.  The routing wave learns it from the route, the
  // second wave by taking the same top-k and table lookup itself before it
  // quantises x.
  const bool early_wg = static_cast<int>(blockIdx.x) < g.nfetch &&
                        static_cast<int>(blockIdx.x) < g.units;
  u32x4 va[4], vb[4];
  int32_t early_e = -1;
  auto early = [&](int32_t e0) {
    early_e = e0;
    if (early_wg && e0 >= 0) {
      const char* src = g.pool + static_cast<int64_t>(e0) * g.rb +
                        static_cast<int64_t>(blockIdx.x) * 16 * g.hidden + wave * 4096 + lane * 16;
#pragma unroll
      for (int h = 0; h < 4; ++h)
        va[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + h * 1024));
    }
  };
  int32_t slot_r;
  bool miss_r;
  if constexpr (UNCACHED)
    route_wave_uncached<PER>(logits, n_experts, top_k, ids, weights, out_slot, fetch_slot,
                             fetch_expert, nmiss_ptr, stats, job_e, job_s, job_k, &job_n, slot_r,
                             miss_r, early);
  else
    route_wave<PER, PERC>(logits, n_experts, top_k, ids, weights, slot_of, slot_expert, stamp,
                          cap, step_ptr, out_slot, fetch_slot, fetch_expert, nmiss_ptr, stats,
                          job_e, job_s, job_k, &job_n, slot_r, miss_r, early);
  if (wave == 0 && lane < top_k) pick_slot[lane] = miss_r ? -1 : slot_r;
  if (wave == 1) {
    // x -> e4m3 codes + per-128 scales in LDS while the first wave routes:
    // every chunk's load first (past the end: x[0] again, ignored)
    constexpr int NC = kGemvMaxHidden / 512;
    uint4 raw[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int i = c * 512 + lane * 8;
      raw[c] = *reinterpret_cast<const uint4*>(x + (i < g.hidden ? i : 0));
    }
    if (early_wg) early(route_first_miss<PER, UNCACHED>(logits, n_experts, top_k, slot_of, step_ptr));
#pragma unroll
    for (int c = 0; c < NC; ++c)
      if (c * 512 < g.hidden) quantize_x8(raw[c], c * 512 + lane * 8 < g.hidden, c * 512 + lane * 8, xq, xs);
  }
  __syncthreads();
  const int I = g.inter;
  if (!UNCACHED && static_cast<int>(blockIdx.x) >= g.nfetch) {
    // hit workgroup (pick k, unit t): gate rows 16t.. (first wave), up rows
    // I + 16t.. (second wave) from the pick's cache slot
    const int hb = static_cast<int>(blockIdx.x) - g.nfetch;
    const int k = hb / g.units;
    const int t = hb - k * g.units;
    if (k >= top_k) return;
    const int32_t s = uniform(pick_slot[k]);
    if (s < 0) return;                       // a miss: a fetch workgroup forms these rows
    const char* rec = g.cache + s * g.rb;
    const int gr = t + wave * g.units;       // the wave's 16-row group of w13
    const uint8_t* base =
        reinterpret_cast<const uint8_t*>(rec) + static_cast<int64_t>(gr) * 16 * g.hidden + lane * 16;
    const float* srow = reinterpret_cast<const float*>(rec + g.off_s13) + (gr >> 3) * g.gb;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    for (int b0 = 0; b0 < g.gb; b0 += kHitChunk) {
      float sw[kHitChunk];
      v8i a[kHitChunk];
#pragma unroll
      for (int c = 0; c < kHitChunk; ++c) sw[c] = srow[min(b0 + c, g.gb - 1)];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < kHitChunk; ++c) a[c] = load_op_nt(base + min(b0 + c, g.gb - 1) * 2048, 1024);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < kHitChunk; ++c) {
        const int b = b0 + c;
        if (b < g.gb) {
          const v4f z = {0.f, 0.f, 0.f, 0.f};
          const v4f d = mfma_e4m3_16x16x128(a[c], load_op32(xq + b * 128 + q * 32), z);
          block_fma(acc, d, sw[c] * xs[b]);
        }
      }
    }
    // every lane of a row group stores its (identical) four up sums
    if (wave == 1) *reinterpret_cast<float4*>(&upsum[4 * q]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    __syncthreads();
    if (wave == 0 && (lane & 15) == 0) {
      const float4 u = *reinterpret_cast<const float4*>(&upsum[4 * q]);
      *reinterpret_cast<float4*>(act + static_cast<int64_t>(k) * I + 16 * t + 4 * q) =
          make_float4(silu_mul(acc[0], u.x), silu_mul(acc[1], u.y), silu_mul(acc[2], u.z),
                      silu_mul(acc[3], u.w));
    }
    return;
  }

  // fetch workgroup b of G.  Its units go round robin (u = b, b + G, ...),
  // as 8 KiB pieces through both waves; then each wave takes the plain
  // bytes (w2, the scales) 4 KiB at a time by ticket (below).
  const int nm = uniform(job_n);
  const int G = g.nfetch;
  const int b = static_cast<int>(blockIdx.x);
  const int U = nm * g.units;
  const int np = 2 * g.kq;                   // pieces per unit (even)
  const int nu = U > b ? (U - 1 - b) / G + 1 : 0;
  const int64_t plain_units = (g.rb - g.w13_bytes) >> 4;   // 16-byte units after w13
  // One piece in flight per workgroup, as in the fetch kernel: the next
  // piece's loads go out once this piece has arrived and its stores are
  // issued, before its MFMAs (and a unit's fold), into the other of two
  // register buffers (a copy between them would wait for the loads just
  // issued).  Issuing them before this piece had arrived (two in flight)
  // made the step 1.3 % slower on MI355X: more outstanding host reads lower
  // the link's rate.  (va, vb: declared with the early read above.)

  // ---- unit pieces: unit u = b + ui * G, pieces p = 0 .. np - 1 (np even,
  // so piece p always lands in buffer p & 1 and a unit's first piece in va)
  auto unit_off = [&](int ui, int p, int& j, int& t) -> int64_t {
    const int u = b + ui * G;
    j = u / g.units;
    t = u - j * g.units;
    const int tw = p / g.kq;
    const int q4 = p - tw * g.kq;
    return static_cast<int64_t>(t + tw * g.units) * 16 * g.hidden +
           static_cast<int64_t>(q4) * kPieceBytes + wave * 4096 + lane * 16;
  };
  // live == false: the same offsets in the device cache, read and ignored.
  // Every load is issued unconditionally: behind a branch, the compiler's
  // wait for the previous piece at the join also covered these loads.
  auto unit_load = [&](int ui, int p, u32x4 (&v)[4], bool live) {
    int j, t;
    const int64_t o = unit_off(ui, p, j, t);
    const char* src = live ? g.pool + uniform(job_e[min(j, nm - 1)]) * g.rb : g.cache;
#pragma unroll
    for (int h = 0; h < 4; ++h)
      v[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + o + h * 1024));
  };
  auto unit_store = [&](int ui, int p, const u32x4 (&v)[4]) {
    int j, t;
    const int64_t o = unit_off(ui, p, j, t);
    char* dst = g.cache + uniform(job_s[j]) * g.rb;
#pragma unroll
    for (int h = 0; h < 4; ++h) *reinterpret_cast<u32x4*>(dst + o + h * 1024) = v[h];
  };
  auto unit_mfma = [&](int p, const u32x4 (&v)[4]) {
    const int tw = p / g.kq;
    const int q4 = p - tw * g.kq;
#pragma unroll
    for (int bl = 0; bl < 2; ++bl) {
      const int gbk = 4 * q4 + 2 * wave + bl;
      const v8i a = {(int)v[2 * bl].x, (int)v[2 * bl].y, (int)v[2 * bl].z, (int)v[2 * bl].w,
                     (int)v[2 * bl + 1].x, (int)v[2 * bl + 1].y, (int)v[2 * bl + 1].z,
                     (int)v[2 * bl + 1].w};
      const v4f z = {0.f, 0.f, 0.f, 0.f};
      const v4f d = mfma_e4m3_16x16x128(a, load_op32(xq + gbk * 128 + q * 32), z);
      // every lane stores: the 16 lanes of a row group hold the same values
      *reinterpret_cast<float4*>(&dpart[tw][gbk][4 * q]) = make_float4(d[0], d[1], d[2], d[3]);
    }
  };
  if (nu > 0 && !(early_wg && early_e >= 0)) unit_load(0, 0, va, true);
  for (int ui = 0; ui < nu; ++ui) {
    int j, t;
    unit_off(ui, 0, j, t);
    // the unit's block scales of this wave's row group (lane c: K-block c),
    // from the host record, for the fold at the unit's end
    const int grw = t + wave * g.units;
    const float sw = reinterpret_cast<const float*>(g.pool + uniform(job_e[j]) * g.rb +
                                                    g.off_s13)[(grw >> 3) * g.gb +
                                                               min(lane, g.gb - 1)];
    for (int p = 0; p < np; p += 2) {
      unit_store(ui, p, va);
      unit_load(ui, p + 1, vb, true);
      unit_mfma(p, va);
      unit_store(ui, p + 1, vb);
      // the unit's next piece, else the next unit's first
      const bool in_unit = p + 2 < np;
      unit_load(in_unit ? ui : ui + 1, in_unit ? p + 2 : 0, va, in_unit || ui + 1 < nu);
      unit_mfma(p + 1, vb);
      if (p == 0) {
        // the scales arrived before the second piece (loads complete in
        // order): parked in LDS here, where no wait is added; read in the
        // fold below, a wait there covers every load in flight
        swl[wave][lane] = sw;
      }
    }
    // wave w folds tile w (gate, up) in K order
    __syncthreads();
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    for (int gbk = 0; gbk < g.gb; ++gbk) {
      const float4 d = *reinterpret_cast<const float4*>(&dpart[wave][gbk][4 * q]);
      const v4f dv = {d.x, d.y, d.z, d.w};
      block_fma(acc, dv, swl[wave][gbk] * xs[gbk]);
    }
    if (wave == 1)
      *reinterpret_cast<float4*>(&upsum[4 * q]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    __syncthreads();
    if (wave == 0 && (lane & 15) == 0) {
      const int kk = uniform(job_k[j]);
      const float4 uu = *reinterpret_cast<const float4*>(&upsum[4 * q]);
      *reinterpret_cast<float4*>(act + static_cast<int64_t>(kk) * I + 16 * t + 4 * q) =
          make_float4(silu_mul(acc[0], uu.x), silu_mul(acc[1], uu.y), silu_mul(acc[2], uu.z),
                      silu_mul(acc[3], uu.w));
    }
  }

  // ---- plain bytes, dealt by ticket: each wave takes 4 KiB pieces (64
  // lanes x 4 x 16 bytes) from the counter the logits launch zeroed, piece
  // gi of job gi / plain (16-byte unit m * 256 + lane + 64 h after w13, the
  // last unit again past the record's end, read and never stored), one in
  // flight, the next ticket requested behind its loads.  Waves whose pieces
  // arrive sooner take more of them, so the fetch ends within about a piece
  // of each wave's last: dealt round robin instead, the workgroups on the
  // XCDs farther from the host link (their first bytes arrive ~3 us later)
  // finished up to 11 us after the others at 8 misses.
  const int P = nm * g.plain;
  auto plain_load = [&](int gi, u32x4 (&v)[4]) {
    const int j = gi / g.plain;
    const int m = gi - j * g.plain;
    const char* src = g.pool + uniform(job_e[j]) * g.rb + g.w13_bytes;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int64_t uidx = min(static_cast<int64_t>(m) * 256 + lane + 64 * h, plain_units - 1);
      v[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + uidx * 16));
    }
  };
  auto plain_store = [&](int gi, const u32x4 (&v)[4]) {
    const int j = gi / g.plain;
    const int m = gi - j * g.plain;
    char* dst = g.cache + uniform(job_s[j]) * g.rb + g.w13_bytes;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int64_t uidx = static_cast<int64_t>(m) * 256 + lane + 64 * h;
      if (uidx < plain_units) *reinterpret_cast<u32x4*>(dst + uidx * 16) = v[h];
    }
  };
  // lane 0's ticket; the other lanes' value is never read
  auto take = [&]() -> int32_t {
    int32_t tk = 0;
    if (lane == 0)
      tk = __hip_atomic_fetch_add(g.ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return tk;
  };
  int32_t tv = take();
  for (int gi = __builtin_amdgcn_readfirstlane(tv); gi < P;
       gi = __builtin_amdgcn_readfirstlane(tv)) {
    plain_load(gi, va);
    tv = take();
    plain_store(gi, va);
  }
}

// The drop-in's fetch + gate/up (moe_fetch_ffn): the reference's four
// buffers per expert (w13, w2 row-major on the host, written in tile order
// to the cache; s13, s2 raw), the miss list from the resolve launch before
// it.  Fetch workgroups take the misses' w13 as units (16 gate + 16 up rows
// of 16 intermediate columns, 2 H/512 tile pieces, each transposed through
// LDS as moe_fetch writes it) and run the gate/up MFMAs on the transposed
// piece in LDS before it is overwritten; the other buffers' pieces are
// plain moe_fetch pieces.  Hit workgroups do a hit's unit from its slot.
// Same arithmetic as route_fetch_gateup_kernel.
//
// RESOLVE (moe_resolve_fetch_ffn): no resolve launch before it; every
// workgroup's first wave makes the call's slot decisions itself from the
// reference's single-buffer table (resolve.hpp, the decisions of
// bin/devcache.py:65-98), which no workgroup of the launch writes:
// workgroup 0 writes the outputs and the table's next state into staging,
// which the down launch copies into the table.
struct ResolveArgs {
  const void* ids;
  int32_t ids64;
  int32_t n_experts;
  const int32_t* slot_of;
  const int32_t* slot_expert;
  const int64_t* stamp;
  const int64_t* step;
  int32_t cap;
  int32_t* next_slot_of;
  int32_t* next_slot_expert;
  int64_t* next_stamp;
  int64_t* next_step;
  int32_t* out_slot;
  int32_t* fetch_slot;
  int32_t* fetch_expert;
  int32_t* nmiss;
  int64_t* stats;
};

template <bool RESOLVE, int PER, int PERC>
__global__ __launch_bounds__(kStepThreads) void fetch_gateup_kernel(
    FetchArgs a, int32_t nfetch, const int32_t* __restrict__ fetch_expert,
    const int32_t* __restrict__ fetch_slot, const int32_t* __restrict__ nmiss_ptr,
    int32_t max_jobs, const int32_t* __restrict__ slots, int32_t top_k,
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ w13c,
    const float* __restrict__ s13c, int64_t w13_es, int64_t s13_es, int32_t n_slots,
    int32_t hidden, int32_t inter, float* __restrict__ act, ResolveArgs ra) {
  __shared__ u32x4 stage[16 * 33];
  __shared__ __align__(16) uint8_t xq[kGemvMaxHidden];
  __shared__ float xs[kGemvMaxHidden / 128];
  __shared__ __align__(16) float dpart[2][kGemvMaxHidden / 128][16];
  __shared__ __align__(16) float upsum[16];
  __shared__ float swl[2][64];
  // job_km[j]: bit k set for every pick k whose slot is job j's (an expert
  // repeated in the row takes one slot for all its picks, and its miss is
  // queued once; every such pick reads the unit's activations)
  __shared__ int32_t job_e[kMaxTopK], job_s[kMaxTopK], job_n;
  __shared__ uint32_t job_km[kMaxTopK];
  __shared__ int32_t pick_slot[kMaxTopK];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4;
  const int gb = hidden / 128;
  const int kq = hidden / 512;
  const int units = inter / 16;
  const uint32_t upr = a.tile_upr[0];      // 16-byte units per w13 row: H / 16
  const int64_t rec0 = a.bytes[0];
  // With RESOLVE, a fetch workgroup whose first unit is of job 0 (b <
  // units) reads that unit's first piece as soon as each wave knows the
  // first miss, before the resolve (which only decides its slot), as
  // route_fetch_gateup_kernel does: the first wave from its lookup, the
  // second from the ids and the table itself.
  const bool early_wg = RESOLVE && static_cast<int>(blockIdx.x) < nfetch &&
                        static_cast<int>(blockIdx.x) < units;
  u32x4 v[4];
  int32_t early_e = -1;
  auto early = [&](int32_t e0) {
    early_e = e0;
    if (early_wg && e0 >= 0) {
      const u32x4* sv = reinterpret_cast<const u32x4*>(a.src[0] + e0 * rec0) +
                        static_cast<int64_t>(blockIdx.x) * 16 * upr;
#pragma unroll
      for (int uu = 0; uu < 4; ++uu) {
        const uint32_t i = threadIdx.x + uu * kStepThreads;
        v[uu] = __builtin_nontemporal_load(sv + (i >> 5) * upr + (i & 31));
      }
    }
  };
  if (wave == 0) {
    if constexpr (RESOLVE) {
      // the table, the step, the counters and the ids in one round trip
      SlotRegs<PERC> t;
      t.load(ra.stamp, ra.slot_expert, ra.cap);
      ExpertRegs<PER> xr;
      xr.load(ra.slot_of, ra.n_experts);
      StatsPrefetch prev;
      prev.load(ra.stats);
      const int64_t step = *ra.step + 1;
      const int li = min(lane, top_k - 1);
      const int64_t e64 = ra.ids64 ? static_cast<const int64_t*>(ra.ids)[li]
                                   : static_cast<int64_t>(static_cast<const int32_t*>(ra.ids)[li]);
      // ids out of range get slot -1 (the down launch poisons their rows)
      const int32_t my_e =
          (lane < top_k && e64 >= 0 && e64 < ra.n_experts) ? static_cast<int32_t>(e64) : -1;
      const int32_t found = xr.lookup(my_e < 0 ? 0 : my_e);
      const int32_t my_s = my_e < 0 ? -1 : found;
      early(first_miss(my_e, my_s));
      int32_t nm = 0;
      int64_t hits = 0;
      int32_t slot_r;
      bool miss_r;
      resolve_regs<PER, PERC>(t, xr, my_e, my_s, top_k, step, ra.cap, job_e, job_s, nullptr, nm,
                              hits, slot_r, miss_r);
      // a pick is formed by the fetch when a miss of this call fills its
      // slot (its own, or an earlier pick's of the same expert)
      bool fetched = false;
      int jn = 0;
      for (int k = 0; k < top_k; ++k) {
        const int32_t mk = __builtin_amdgcn_readlane(miss_r ? 1 : 0, k);
        const int32_t sk = __builtin_amdgcn_readlane(slot_r, k);
        if (mk) {
          const uint64_t b = __ballot(lane < top_k && slot_r == sk);
          if (lane == 0) job_km[jn] = static_cast<uint32_t>(b);
          fetched |= slot_r == sk;
          ++jn;
        }
      }
      if (lane < top_k) pick_slot[lane] = (slot_r < 0 || fetched) ? -1 : slot_r;
      if (lane == 0) job_n = nm;
      if (blockIdx.x == 0) {
        if (lane < top_k) ra.out_slot[lane] = slot_r;
#pragma unroll
        for (int j = 0; j < PERC; ++j) {
          const int c = lane + 64 * j;
          if (c < ra.cap) {
            ra.next_stamp[c] = t.st[j];
            ra.next_slot_expert[c] = t.se[j];
          }
        }
#pragma unroll
        for (int j = 0; j < PER; ++j) {
          const int e = lane + 64 * j;
          if (e < ra.n_experts) ra.next_slot_of[e] = xr.so[j];
        }
        if (lane == 0) {
          for (int j = 0; j < nm; ++j) {
            ra.fetch_expert[j] = job_e[j];
            ra.fetch_slot[j] = job_s[j];
          }
          *ra.next_step = step;
          *ra.nmiss = nm;
          if (ra.stats) {
            ra.stats[0] = prev.hits + hits;
            ra.stats[1] = prev.misses + nm;
          }
        }
      }
    } else {
      // the miss list and the picks' slots; a pick missed when its slot is in
      // the list (a repeated expert's picks all did)
      const int nm = min(*nmiss_ptr, max_jobs);
      const int32_t fe = fetch_expert[min(lane, max_jobs - 1)];
      const int32_t fs = fetch_slot[min(lane, max_jobs - 1)];
      const int32_t sl = slots[min(lane, top_k - 1)];
      bool miss = false;
      uint32_t km = 0;
      for (int j = 0; j < nm; ++j) miss |= __builtin_amdgcn_readlane(fs, j) == sl;
      for (int k = 0; k < top_k; ++k)
        if (__builtin_amdgcn_readlane(sl, k) == fs) km |= 1u << k;
      if (lane < nm) {
        job_e[lane] = fe;
        job_s[lane] = fs;
        job_km[lane] = km;
      }
      if (lane < top_k) pick_slot[lane] = miss ? -1 : sl;
      if (lane == 0) job_n = nm;
    }
  } else {
    constexpr int NC = kGemvMaxHidden / 512;
    uint4 raw[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int i = c * 512 + lane * 8;
      raw[c] = *reinterpret_cast<const uint4*>(x + (i < hidden ? i : 0));
    }
    if (early_wg) {
      // the first miss: the first pick absent from the table
      ExpertRegs<PER> xr;
      xr.load(ra.slot_of, ra.n_experts);
      const int li = min(lane, top_k - 1);
      const int64_t e64 = ra.ids64 ? static_cast<const int64_t*>(ra.ids)[li]
                                   : static_cast<int64_t>(static_cast<const int32_t*>(ra.ids)[li]);
      const int32_t my_e =
          (lane < top_k && e64 >= 0 && e64 < ra.n_experts) ? static_cast<int32_t>(e64) : -1;
      const int32_t found = xr.lookup(my_e < 0 ? 0 : my_e);
      early(first_miss(my_e, my_e < 0 ? -1 : found));
    }
#pragma unroll
    for (int c = 0; c < NC; ++c)
      if (c * 512 < hidden) quantize_x8(raw[c], c * 512 + lane * 8 < hidden, c * 512 + lane * 8, xq, xs);
  }
  __syncthreads();
  if (static_cast<int>(blockIdx.x) >= nfetch) {
    const int hb = static_cast<int>(blockIdx.x) - nfetch;
    const int k = hb / units;
    const int t = hb - k * units;
    if (k >= top_k) return;
    const int32_t s = uniform(pick_slot[k]);
    // a miss, or no such slot (the down launch poisons that pick's output)
    if (s < 0 || s >= n_slots) return;
    const int gr = t + wave * units;
    const uint8_t* base = w13c + s * w13_es + static_cast<int64_t>(gr) * 16 * hidden + lane * 16;
    const float* srow = s13c + s * s13_es + (gr >> 3) * gb;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    for (int b0 = 0; b0 < gb; b0 += kHitChunk) {
      float sw[kHitChunk];
      v8i av[kHitChunk];
#pragma unroll
      for (int c = 0; c < kHitChunk; ++c) sw[c] = srow[min(b0 + c, gb - 1)];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < kHitChunk; ++c) av[c] = load_op_nt(base + min(b0 + c, gb - 1) * 2048, 1024);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < kHitChunk; ++c) {
        const int b = b0 + c;
        if (b < gb) {
          const v4f z = {0.f, 0.f, 0.f, 0.f};
          const v4f dd = mfma_e4m3_16x16x128(av[c], load_op32(xq + b * 128 + q * 32), z);
          block_fma(acc, dd, sw[c] * xs[b]);
        }
      }
    }
    if (wave == 1) *reinterpret_cast<float4*>(&upsum[4 * q]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    __syncthreads();
    if (wave == 0 && (lane & 15) == 0) {
      const float4 u = *reinterpret_cast<const float4*>(&upsum[4 * q]);
      *reinterpret_cast<float4*>(act + static_cast<int64_t>(k) * inter + 16 * t + 4 * q) =
          make_float4(silu_mul(acc[0], u.x), silu_mul(acc[1], u.y), silu_mul(acc[2], u.z),
                      silu_mul(acc[3], u.w));
    }
    return;
  }
  // fetch workgroup b of G: its units (round robin), then its plain pieces
  // (those of the buffers after w13: first 8 to each workgroup with one unit
  // fewer, then round robin), as in route_fetch_gateup_kernel
  const int nm = uniform(job_n);
  const int G = nfetch;
  const int b = static_cast<int>(blockIdx.x);
  const int U = nm * units;
  const int plain = static_cast<int>(a.pieces_per_job - a.pieces[0]);
  const int P = nm * plain;
  const int r = U % G;
  const int A = r > 0 ? min(P, 8 * (G - r)) : 0;
  const int np = 2 * kq;
  const int nu = U > b ? (U - 1 - b) / G + 1 : 0;
  // unit piece p of the workgroup's unit ui: its host rows (lane's loads) and
  // its cache run; live == false reads the same offsets of the cache (the
  // loads stay unconditional: behind a branch, the compiler's wait at the
  // join would cover them)
  auto piece_src = [&](int ui, int p, bool live) -> const u32x4* {
    const int u = b + ui * G;
    const int j = u / units;
    const int t = u - j * units;
    const int tw = p / kq;
    const int q4 = p - tw * kq;
    const uint32_t g16 = static_cast<uint32_t>(t + tw * units);
    const char* base = live ? a.src[0] + uniform(job_e[min(j, nm - 1)]) * rec0 : a.dst[0];
    return reinterpret_cast<const u32x4*>(base) + static_cast<int64_t>(g16) * 16 * upr + q4 * 32;
  };
  auto load_piece = [&](const u32x4* sv, u32x4 (&v)[4]) {
#pragma unroll
    for (int uu = 0; uu < 4; ++uu) {
      const uint32_t i = threadIdx.x + uu * kStepThreads;
      v[uu] = __builtin_nontemporal_load(sv + (i >> 5) * upr + (i & 31));
    }
  };
  if (nu > 0 && !(early_wg && early_e >= 0)) load_piece(piece_src(0, 0, true), v);
  for (int ui = 0; ui < nu; ++ui) {
    const int u = b + ui * G;
    const int j = u / units;
    const int t = u - j * units;
    const int32_t e = uniform(job_e[j]);
    const int32_t s = uniform(job_s[j]);
    const int grw = t + wave * units;
    const float sw = reinterpret_cast<const float*>(a.src[2] + e * a.bytes[2])[(grw >> 3) * gb +
                                                                              min(lane, gb - 1)];
    u32x4* dstv = reinterpret_cast<u32x4*>(a.dst[0] + s * rec0);
    for (int p = 0; p < np; ++p) {
      const int tw = p / kq;
      const int q4 = p - tw * kq;
      const uint32_t g16 = static_cast<uint32_t>(t + tw * units);   // 16-row group of w13
      u32x4* dv = dstv + (static_cast<int64_t>(g16) * upr + q4 * 32) * 16;
#pragma unroll
      for (int uu = 0; uu < 4; ++uu) {
        const uint32_t i = threadIdx.x + uu * kStepThreads;
        stage[(i >> 5) * 33 + (i & 31)] = v[uu];
      }
      __syncthreads();
      // the piece is in LDS: the next one's loads go out now, into the same
      // registers, while this one is stored and multiplied (one piece in
      // flight per workgroup, as in the fetch kernel)
      {
        const bool in_unit = p + 1 < np;
        load_piece(piece_src(in_unit ? ui : ui + 1, in_unit ? p + 1 : 0, in_unit || ui + 1 < nu),
                   v);
      }
#pragma unroll
      for (int uu = 0; uu < 4; ++uu) {
        // destination unit dd = (2 bb + h) * 64 + 16 qq + rr: row rr, column unit 8 bb + 2 qq + h
        const uint32_t dd = threadIdx.x + uu * kStepThreads;
        const uint32_t bh = dd >> 6, qq = (dd >> 4) & 3, rr = dd & 15;
        dv[dd] = stage[rr * 33 + (bh >> 1) * 8 + 2 * qq + (bh & 1)];
      }
      // this wave's K-blocks 2 wave, 2 wave + 1 of the piece: A from the
      // transposed rows in LDS (lane 16q + r: row r, units 8 bl + 2q, + 1)
#pragma unroll
      for (int bl2 = 0; bl2 < 2; ++bl2) {
        const int bl = 2 * wave + bl2;
        const u32x4 lo = stage[(lane & 15) * 33 + 8 * bl + 2 * q];
        const u32x4 hi = stage[(lane & 15) * 33 + 8 * bl + 2 * q + 1];
        const v8i av = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                        (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        const int gbk = 4 * q4 + bl;
        const v4f z = {0.f, 0.f, 0.f, 0.f};
        const v4f dd = mfma_e4m3_16x16x128(av, load_op32(xq + gbk * 128 + q * 32), z);
        *reinterpret_cast<float4*>(&dpart[tw][gbk][4 * q]) = make_float4(dd[0], dd[1], dd[2], dd[3]);
      }
      if (p == 0) swl[wave][lane] = sw;
      __syncthreads();
    }
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    for (int gbk = 0; gbk < gb; ++gbk) {
      const float4 dd = *reinterpret_cast<const float4*>(&dpart[wave][gbk][4 * q]);
      const v4f dv = {dd.x, dd.y, dd.z, dd.w};
      block_fma(acc, dv, swl[wave][gbk] * xs[gbk]);
    }
    if (wave == 1)
      *reinterpret_cast<float4*>(&upsum[4 * q]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    __syncthreads();
    if (wave == 0 && (lane & 15) == 0) {
      uint32_t km = static_cast<uint32_t>(uniform(static_cast<int32_t>(job_km[j])));
      const float4 uu = *reinterpret_cast<const float4*>(&upsum[4 * q]);
      const float4 av = make_float4(silu_mul(acc[0], uu.x), silu_mul(acc[1], uu.y),
                                    silu_mul(acc[2], uu.z), silu_mul(acc[3], uu.w));
      // a queued slot no pick names (a caller's stale list) writes nothing
      while (km) {
        const int kk = __builtin_ctz(km);
        km &= km - 1;
        *reinterpret_cast<float4*>(act + static_cast<int64_t>(kk) * inter + 16 * t + 4 * q) = av;
      }
    }
    __syncthreads();
  }
  const int na = (r > 0 && b >= r && A > b - r) ? (A - 1 - (b - r)) / (G - r) + 1 : 0;
  const int nb = P > A + b ? (P - 1 - A - b) / G + 1 : 0;
  for (int n = 0; n < na + nb; ++n) {
    const int gi = n < na ? (b - r) + n * (G - r) : A + b + (n - na) * G;
    const int j = gi / plain;
    fetch_piece(a, a.pieces[0] + (gi - j * plain), uniform(job_e[j]), uniform(job_s[j]), stage);
  }
}

// Events armed by moe_time_fused_launch for the calling thread's next fused
// fetch + gate/up launch (hipExtLaunchKernel records them around that one
// dispatch); taken, and so disarmed, by the next moe_route_fetch_ffn or
// moe_fetch_ffn call whether or not it launches.
thread_local hipEvent_t t_fused_start = nullptr;
thread_local hipEvent_t t_fused_stop = nullptr;

inline void take_fused_events(hipEvent_t& e0, hipEvent_t& e1) {
  e0 = t_fused_start;
  e1 = t_fused_stop;
  t_fused_start = t_fused_stop = nullptr;
}

}  // namespace moe

using namespace moe;

extern "C" int moe_time_fused_launch(void* start, void* stop) {
  MOE_REQUIRE((start == nullptr) == (stop == nullptr),
              "moe_time_fused_launch: give both events or neither");
  t_fused_start = static_cast<hipEvent_t>(start);
  t_fused_stop = static_cast<hipEvent_t>(stop);
  return MOE_OK;
}

// moe_route_fetch_ffn and, with no slot table (slot_of, slot_expert,
// slot_stamp and step NULL), moe_route_fetch_ffn_uncached: the checks and
// the three launches.
static int route_fetch_ffn_impl(const char* fn, bool uncached, const void* x, const void* w,
                                const float* bias, int32_t logit_dtype, int32_t hidden,
                                int32_t n_experts, int32_t top_k, float* logits, int32_t* ids,
                                float* weights, int32_t* slot_of, int32_t* slot_expert,
                                int64_t* slot_stamp, int32_t cap, int64_t* step,
                                int32_t* out_slot, int32_t* fetch_slot, int32_t* fetch_expert,
                                int32_t* nmiss, int64_t* stats, const void* pool, void* cache,
                                int64_t record_bytes, int32_t inter, int32_t blocks_per_job,
                                const moe_shared_expert* shared, const void* residual, void* out,
                                void* workspace, size_t workspace_bytes, void* stream) {
  hipEvent_t ev0, ev1;
  take_fused_events(ev0, ev1);
  MOE_REQUIRE(x && w && logits && ids && weights && out_slot && fetch_slot && fetch_expert &&
                  nmiss && pool && cache && out && workspace,
              "%s: NULL pointer", fn);
  MOE_REQUIRE(uncached || (slot_of && slot_expert && slot_stamp && step), "%s: NULL pointer", fn);
  MOE_REQUIRE(logit_dtype == MOE_F32 || logit_dtype == MOE_BF16,
              "%s: logit_dtype must be MOE_F32 or MOE_BF16", fn);
  MOE_REQUIRE(hidden >= 512 && hidden % 512 == 0 && hidden <= kGemvMaxHidden,
              "%s: hidden must be a multiple of 512 up to %d (got %d)", fn, kGemvMaxHidden, hidden);
  MOE_REQUIRE(inter >= 128 && inter % 128 == 0 && inter <= kGemvMaxInter,
              "%s: inter must be a multiple of 128 up to %d (got %d)", fn, kGemvMaxInter, inter);
  MOE_REQUIRE(top_k >= 1 && top_k <= kGemvMaxTopK && top_k <= n_experts && n_experts <= 1024,
              "%s: need 1 <= top_k <= min(%d, n_experts), n_experts <= 1024", fn, kGemvMaxTopK);
  MOE_REQUIRE(cap >= 1 && cap <= 1024, "%s: need 1 <= cap <= 1024", fn);
  MOE_REQUIRE(top_k <= cap, "%s: top_k (%d) exceeds the cache capacity (%d)", fn, top_k, cap);
  const int64_t w13 = 2LL * inter * hidden;
  const int64_t off_s13 = w13 + static_cast<int64_t>(hidden) * inter;
  const int64_t off_s2 = off_s13 + (2LL * inter / 128) * (hidden / 128) * 4;
  const int64_t payload = off_s2 + (static_cast<int64_t>(hidden) / 128) * (inter / 128) * 4;
  MOE_REQUIRE(record_bytes >= payload && record_bytes % 256 == 0,
              "%s: record_bytes (%lld) must hold the %lld-byte record and be a multiple of 256",
              fn, (long long)record_bytes, (long long)payload);
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(pool) % 256 == 0 &&
                  reinterpret_cast<uintptr_t>(cache) % 256 == 0,
              "%s: pool and cache must be 256-byte aligned", fn);
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0,
              "%s: x and w must be 16-byte aligned", fn);
  // workspace: act [top_k, inter] f32 from byte 0, the fetch's piece
  // counter (int32) at the next 256-byte boundary; with the shared expert,
  // its act [Is] bf16 and sig f32 after them (moe_fp8_moe_block_forward's
  // layout for one token, from moe_fp8_moe_workspace(1, ...) >= 8 top_k
  // inter bytes, past the counter since top_k inter >= 128)
  const size_t base = (moe_fp8_moe_workspace(1, top_k, cap, hidden, inter) + 255) & ~size_t{255};
  const size_t act_bytes = (static_cast<size_t>(top_k) * inter * sizeof(float) + 255) & ~size_t{255};
  size_t need = act_bytes + 256;
  SharedRefs sh{};
  if (shared) {
    const int32_t Is = shared->inter;
    MOE_REQUIRE(Is >= 128 && Is % 128 == 0,
                "%s: shared inter must be a positive multiple of 128", fn);
    MOE_REQUIRE(shared->w_gate && shared->w_up && shared->w_down && shared->w_sgate,
                "%s: NULL shared expert weight", fn);
    MOE_REQUIRE(reinterpret_cast<uintptr_t>(shared->w_gate) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(shared->w_up) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(shared->w_down) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(shared->w_sgate) % 16 == 0,
                "%s: shared expert weights must be 16-byte aligned", fn);
    need = moe_fp8_moe_block_workspace(1, top_k, cap, hidden, inter, Is);
    char* ws = static_cast<char*>(workspace);
    sh = SharedRefs{static_cast<const uint16_t*>(shared->w_gate),
                    static_cast<const uint16_t*>(shared->w_up),
                    static_cast<const uint16_t*>(shared->w_down),
                    static_cast<const uint16_t*>(shared->w_sgate), Is,
                    reinterpret_cast<uint16_t*>(ws + base),
                    reinterpret_cast<float*>(ws + base + ((static_cast<size_t>(Is) * 2 + 255) &
                                                          ~size_t{255}))};
  }
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0 && workspace_bytes >= need,
              "%s: the workspace must be 256-byte aligned and hold %zu bytes (%zu given)", fn,
              need, workspace_bytes);
  MOE_REQUIRE(blocks_per_job >= 1 && blocks_per_job <= 4096,
              "%s: need 1 <= blocks_per_job <= 4096", fn);
  hipStream_t s = as_stream(stream);
  int32_t* ticket = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + act_bytes);
  int rc = launch_decode_logits(x, w, bias, hidden, n_experts, logit_dtype == MOE_BF16 ? 1 : 0,
                                logits, step, s, ticket);
  if (rc) return rc;
  StepGeom g;
  g.ticket = ticket;
  g.pool = static_cast<const char*>(pool);
  g.cache = static_cast<char*>(cache);
  g.rb = record_bytes;
  g.w13_bytes = w13;
  g.off_s13 = off_s13;
  g.hidden = hidden;
  g.inter = inter;
  g.gb = hidden / 128;
  g.kq = hidden / 512;
  g.units = inter / 16;
  g.plain = static_cast<int32_t>((record_bytes - w13 + 4095) / 4096);
  g.nfetch = blocks_per_job * (top_k < kFetchMaxJobsInGrid ? top_k : kFetchMaxJobsInGrid);
  const int nshared = shared ? (shared->inter + 1 + 2 * kSharedJPW - 1) / (2 * kSharedJPW) : 0;
  const unsigned grid =
      static_cast<unsigned>(g.nfetch + (uncached ? 0 : top_k * g.units) + nshared);
  float* act = static_cast<float*>(workspace);
#define MOE_RFG(U, PE, PC)                                                                     \
  hipExtLaunchKernelGGL((route_fetch_gateup_kernel<U, PE, PC>), dim3(grid), dim3(kStepThreads),  \
                        0, s, ev0, ev1, 0, g, static_cast<const uint16_t*>(x), logits, n_experts, \
                        top_k, ids, weights, slot_of, slot_expert, slot_stamp, cap, step,        \
                        out_slot, fetch_slot, fetch_expert, nmiss, stats, act, sh)
  if (uncached) {
    if (n_experts <= 256) MOE_RFG(true, 4, 4); else MOE_RFG(true, 16, 4);
  } else if (n_experts <= 256) {
    if (cap <= 256) MOE_RFG(false, 4, 4); else MOE_RFG(false, 4, 16);
  } else {
    if (cap <= 256) MOE_RFG(false, 16, 4); else MOE_RFG(false, 16, 16);
  }
#undef MOE_RFG
  rc = check_launch(fn);
  if (rc) return rc;
  const uint8_t* cb = static_cast<const uint8_t*>(cache);
  return launch_down_gemv(act, out_slot, weights, 0, 1, top_k, cb + w13,
                          reinterpret_cast<const float*>(cb + off_s2), record_bytes,
                          record_bytes / 4, MOE_LAYOUT_TILES, cap, hidden, inter,
                          static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(out),
                          shared ? &sh : nullptr, s);
}

extern "C" int moe_route_fetch_ffn(const void* x, const void* w, const float* bias,
                                   int32_t logit_dtype, int32_t hidden, int32_t n_experts,
                                   int32_t top_k, float* logits, int32_t* ids, float* weights,
                                   int32_t* slot_of, int32_t* slot_expert, int64_t* slot_stamp,
                                   int32_t cap, int64_t* step, int32_t* out_slot,
                                   int32_t* fetch_slot, int32_t* fetch_expert, int32_t* nmiss,
                                   int64_t* stats, const void* pool, void* cache,
                                   int64_t record_bytes, int32_t inter, int32_t blocks_per_job,
                                   const moe_shared_expert* shared, const void* residual,
                                   void* out, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  return route_fetch_ffn_impl("moe_route_fetch_ffn", false, x, w, bias, logit_dtype, hidden,
                              n_experts, top_k, logits, ids, weights, slot_of, slot_expert,
                              slot_stamp, cap, step, out_slot, fetch_slot, fetch_expert, nmiss,
                              stats, pool, cache, record_bytes, inter, blocks_per_job, shared,
                              residual, out, workspace, workspace_bytes, stream);
}

extern "C" int moe_route_fetch_ffn_uncached(
    const void* x, const void* w, const float* bias, int32_t logit_dtype, int32_t hidden,
    int32_t n_experts, int32_t top_k, float* logits, int32_t* ids, float* weights,
    int32_t cap, int32_t* out_slot, int32_t* fetch_slot, int32_t* fetch_expert, int32_t* nmiss,
    int64_t* stats, const void* pool, void* cache, int64_t record_bytes, int32_t inter,
    int32_t blocks_per_job, const moe_shared_expert* shared, const void* residual, void* out,
    void* workspace, size_t workspace_bytes, void* stream) {
  return route_fetch_ffn_impl("moe_route_fetch_ffn_uncached", true, x, w, bias, logit_dtype,
                              hidden, n_experts, top_k, logits, ids, weights, nullptr, nullptr,
                              nullptr, cap, nullptr, out_slot, fetch_slot, fetch_expert, nmiss,
                              stats, pool, cache, record_bytes, inter, blocks_per_job, shared,
                              residual, out, workspace, workspace_bytes, stream);
}

// The checks moe_fetch_ffn and moe_resolve_fetch_ffn share: the four buffer
// pairs against the cache buffers and the shapes the kernels take; fills a.
static int fetch_ffn_checks(const char* what, const moe_fetch_pair* pairs, int32_t npairs,
                            int32_t max_jobs, int32_t blocks_per_job, const void* x,
                            int32_t w_dtype, int32_t top_k, const void* w13, const float* s13,
                            const void* w2, const float* s2, int32_t n_slots, int32_t hidden,
                            int32_t inter, const moe_expert_strides* strides, void* workspace,
                            size_t workspace_bytes, FetchArgs* a) {
  MOE_REQUIRE(npairs == 4, "%s: takes the four buffers w13, w2, s13, s2 (got %d)", what, npairs);
  MOE_REQUIRE(w_dtype == MOE_F32 || w_dtype == MOE_BF16,
              "%s: w_dtype must be MOE_F32 or MOE_BF16", what);
  MOE_REQUIRE(hidden >= 512 && hidden % 512 == 0 && hidden <= kGemvMaxHidden,
              "%s: hidden must be a multiple of 512 up to %d (got %d)", what, kGemvMaxHidden,
              hidden);
  MOE_REQUIRE(inter >= 128 && inter % 128 == 0 && inter <= kGemvMaxInter,
              "%s: inter must be a multiple of 128 up to %d (got %d)", what, kGemvMaxInter, inter);
  MOE_REQUIRE(top_k >= 1 && top_k <= kGemvMaxTopK && top_k <= n_slots && n_slots >= 1,
              "%s: need 1 <= top_k <= min(%d, n_slots)", what, kGemvMaxTopK);
  MOE_REQUIRE(max_jobs >= top_k && max_jobs <= kMaxTopK, "%s: need top_k <= max_jobs <= %d",
              what, kMaxTopK);
  MOE_REQUIRE(strides->layout == MOE_LAYOUT_TILES, "%s: the cache must hold w13/w2 in tile order",
              what);
  const int64_t w13b = 2LL * inter * hidden;
  const int64_t s13b = (2LL * inter / 128) * (hidden / 128) * 4;
  const int64_t w2b = static_cast<int64_t>(hidden) * inter;
  const int64_t s2b = (static_cast<int64_t>(hidden) / 128) * (inter / 128) * 4;
  MOE_REQUIRE(pairs[0].bytes == w13b && pairs[0].tile_k == hidden,
              "%s: pair 0 must be w13 (%lld bytes, tile_k = hidden)", what, (long long)w13b);
  MOE_REQUIRE(pairs[1].bytes == w2b && pairs[1].tile_k == inter,
              "%s: pair 1 must be w2 (tile_k = inter)", what);
  MOE_REQUIRE(pairs[2].bytes == s13b && pairs[2].tile_k == 0,
              "%s: pair 2 must be s13 (%lld bytes, a byte copy)", what, (long long)s13b);
  MOE_REQUIRE(pairs[3].bytes == s2b && pairs[3].tile_k == 0,
              "%s: pair 3 must be s2 (%lld bytes, a byte copy)", what, (long long)s2b);
  MOE_REQUIRE(pairs[0].dst == w13 && pairs[2].dst == s13 && strides->w13 == w13b &&
                  strides->s13 == s13b / 4,
              "%s: the w13 and s13 pairs must fill the cache buffers w13 and s13 (dense, one "
              "expert after another)", what);
  MOE_REQUIRE(pairs[1].dst == w2 && pairs[3].dst == s2 && strides->w2 == w2b &&
                  strides->s2 == s2b / 4,
              "%s: the w2 and s2 pairs must fill the cache buffers w2 and s2 (dense, one expert "
              "after another)", what);
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0, "%s: x must be 16-byte aligned", what);
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                  workspace_bytes >= static_cast<size_t>(top_k) * inter * sizeof(float),
              "%s: the workspace must be 16-byte aligned and hold top_k * inter floats", what);
  MOE_REQUIRE(blocks_per_job >= 1 && blocks_per_job <= 4096,
              "%s: need 1 <= blocks_per_job <= 4096", what);
  const int rc0 = fetch_args(pairs, npairs, max_jobs, a);
  if (rc0 != MOE_OK) return rc0;
  MOE_REQUIRE(a->tile_wlog[0] == 5, "%s: w13 pieces must be 32 column units wide", what);
  return MOE_OK;
}

extern "C" int moe_fetch_ffn(const moe_fetch_pair* pairs, int32_t npairs,
                             const int32_t* fetch_expert, const int32_t* fetch_slot,
                             const int32_t* nmiss, int32_t max_jobs, int32_t blocks_per_job,
                             const void* x, const int32_t* slots, const void* weights,
                             int32_t w_dtype, int32_t top_k, const void* w13, const float* s13,
                             const void* w2, const float* s2, int32_t n_slots, int32_t hidden,
                             int32_t inter, const moe_expert_strides* strides,
                             const void* residual, void* out, void* workspace,
                             size_t workspace_bytes, void* stream) {
  hipEvent_t ev0, ev1;
  take_fused_events(ev0, ev1);
  MOE_REQUIRE(pairs && fetch_expert && fetch_slot && nmiss && x && slots && weights && w13 &&
                  s13 && w2 && s2 && strides && out && workspace,
              "moe_fetch_ffn: NULL pointer");
  FetchArgs a;
  const int rc0 = fetch_ffn_checks("moe_fetch_ffn", pairs, npairs, max_jobs, blocks_per_job, x,
                                   w_dtype, top_k, w13, s13, w2, s2, n_slots, hidden, inter,
                                   strides, workspace, workspace_bytes, &a);
  if (rc0 != MOE_OK) return rc0;
  hipStream_t s = as_stream(stream);
  const int nfetch = blocks_per_job * (max_jobs < kFetchMaxJobsInGrid ? max_jobs : kFetchMaxJobsInGrid);
  float* act = static_cast<float*>(workspace);
  hipExtLaunchKernelGGL((fetch_gateup_kernel<false, 4, 4>), dim3(nfetch + top_k * (inter / 16)),
                        dim3(kStepThreads), 0, s, ev0, ev1, 0, a, nfetch, fetch_expert, fetch_slot,
                        nmiss, max_jobs, slots, top_k, static_cast<const uint16_t*>(x),
                        static_cast<const uint8_t*>(w13), s13, strides->w13, strides->s13, n_slots,
                        hidden, inter, act, ResolveArgs{});
  const int rc = check_launch("moe_fetch_ffn(fetch+gate/up)");
  if (rc) return rc;
  return launch_down_gemv(act, slots, weights, w_dtype == MOE_BF16 ? 1 : 0, 1, top_k,
                          static_cast<const uint8_t*>(w2), s2, strides->w2, strides->s2,
                          MOE_LAYOUT_TILES, n_slots, hidden, inter,
                          static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(out),
                          nullptr, s);
}

extern "C" int moe_resolve_fetch_ffn(const void* ids, int32_t ids_dtype, int32_t top_k,
                                     const moe_slot_table* table, int32_t* out_slot,
                                     int32_t* fetch_slot, int32_t* fetch_expert, int32_t* nmiss,
                                     int64_t* stats, const moe_fetch_pair* pairs, int32_t npairs,
                                     int32_t blocks_per_job, const void* x, const void* weights,
                                     int32_t w_dtype, const void* w13, const float* s13,
                                     const void* w2, const float* s2, int32_t hidden,
                                     int32_t inter, const moe_expert_strides* strides,
                                     const void* residual, void* out, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  hipEvent_t ev0, ev1;
  take_fused_events(ev0, ev1);
  MOE_REQUIRE(ids && table && out_slot && fetch_slot && fetch_expert && nmiss && pairs && x &&
                  weights && w13 && s13 && w2 && s2 && strides && out && workspace,
              "moe_resolve_fetch_ffn: NULL pointer");
  MOE_REQUIRE(ids_dtype == MOE_I32 || ids_dtype == MOE_I64,
              "moe_resolve_fetch_ffn: ids_dtype must be MOE_I32 or MOE_I64");
  const moe_slot_table& tb = *table;
  MOE_REQUIRE(tb.slot_of && tb.slot_expert && tb.stamp && tb.step && tb.next_slot_of &&
                  tb.next_slot_expert && tb.next_stamp && tb.next_step,
              "moe_resolve_fetch_ffn: NULL table or staging pointer");
  MOE_REQUIRE(tb.n_experts >= 1 && tb.n_experts <= 1024,
              "moe_resolve_fetch_ffn: need 1 <= n_experts <= 1024 (got %d)", tb.n_experts);
  MOE_REQUIRE(tb.cap >= 1 && tb.cap <= 1024, "moe_resolve_fetch_ffn: need 1 <= cap <= 1024");
  MOE_REQUIRE(top_k <= tb.cap, "moe_resolve_fetch_ffn: top_k (%d) exceeds the cache capacity (%d)",
              top_k, tb.cap);
  MOE_REQUIRE(tb.next_slot_of != tb.slot_of && tb.next_slot_expert != tb.slot_expert &&
                  tb.next_stamp != tb.stamp && tb.next_step != tb.step,
              "moe_resolve_fetch_ffn: the staging buffers must not be the table's");
  FetchArgs a;
  const int rc0 = fetch_ffn_checks("moe_resolve_fetch_ffn", pairs, npairs, top_k, blocks_per_job,
                                   x, w_dtype, top_k, w13, s13, w2, s2, tb.cap, hidden, inter,
                                   strides, workspace, workspace_bytes, &a);
  if (rc0 != MOE_OK) return rc0;
  hipStream_t s = as_stream(stream);
  const int nfetch = blocks_per_job * (top_k < kFetchMaxJobsInGrid ? top_k : kFetchMaxJobsInGrid);
  float* act = static_cast<float*>(workspace);
  ResolveArgs ra{ids, ids_dtype == MOE_I64 ? 1 : 0, tb.n_experts, tb.slot_of, tb.slot_expert,
                 tb.stamp, tb.step, tb.cap, tb.next_slot_of, tb.next_slot_expert, tb.next_stamp,
                 tb.next_step, out_slot, fetch_slot, fetch_expert, nmiss, stats};
  const dim3 grid(nfetch + top_k * (inter / 16));
#define MOE_RFF(PE, PC)                                                                       \
  hipExtLaunchKernelGGL((fetch_gateup_kernel<true, PE, PC>), grid, dim3(kStepThreads), 0, s,  \
                        ev0, ev1, 0, a, nfetch, fetch_expert, fetch_slot, nmiss, top_k,      \
                        out_slot, top_k, static_cast<const uint16_t*>(x),                     \
                        static_cast<const uint8_t*>(w13), s13, strides->w13, strides->s13,   \
                        tb.cap, hidden, inter, act, ra)
  if (tb.n_experts <= 256) {
    if (tb.cap <= 256) MOE_RFF(4, 4); else MOE_RFF(4, 16);
  } else {
    if (tb.cap <= 256) MOE_RFF(16, 4); else MOE_RFF(16, 16);
  }
#undef MOE_RFF
  const int rc = check_launch("moe_resolve_fetch_ffn(resolve+fetch+gate/up)");
  if (rc) return rc;
  // the down launch reads the slots written above and copies the staged
  // table into the table
  const TableCommit cm{tb.next_slot_of, tb.slot_of, tb.next_slot_expert, tb.slot_expert,
                       tb.next_stamp, tb.stamp, tb.next_step, tb.step, tb.n_experts, tb.cap};
  return launch_down_gemv(act, out_slot, weights, w_dtype == MOE_BF16 ? 1 : 0, 1, top_k,
                          static_cast<const uint8_t*>(w2), s2, strides->w2, strides->s2,
                          MOE_LAYOUT_TILES, tb.cap, hidden, inter,
                          static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(out),
                          nullptr, s, &cm);
}
