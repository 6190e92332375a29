// W8A8 block-FP8 expert FFN, per (token, expert) pair: the decode GEMV path.
//
// For pair p = t*K + k with expert e = ids[p]:
//   xq, xs = e4m3 quantisation of x[t], per 128 columns, scale amax/448
//   h[p][r] = sum_g s13[e][r/128][g] * xs[g] * <w13[e][r][g*128:+128], xq[g*128:+128]>
//   a = SiLU(h[:I]) * h[I:], quantised per 128 (aq, as)
//   y[c]    = sum_g s2[e][c/128][g] * as[g] * <w2[e][c][g*128:+128], aq[g*128:+128]>
//   out[t]  = fma(w[t][k], y_k, out[t]) for k in order, float32 -> bf16
//
// Each 128-term block product runs on one v_mfma_scale_f32_16x16x128_f8f6f4
// with the weight rows as the A operand (16 rows per wave) and the quantised
// activation as every column of B; column 0 of the result is used.  Weights
// are read straight from HBM into the A registers: each lane reads 32
// contiguous bytes of its row per block, so a wave reads 16 rows x 128 B,
// whole cache lines.  The block scales multiply the fp32 block result, so the
// scale of every 128x128 weight block is applied exactly once per block.
//
// Kernel 1 (gate/up + SiLU): grid (I/16, pairs), four waves per workgroup:
// gate rows 16j..16j+15 and the up rows I+16j.. of the same intermediate
// columns, each tile split over K between two waves, x quantised into LDS by
// the four together; the workgroup ends with a = SiLU(gate) * up of its 16
// columns (float32, the pair's row of the workspace).  Kernel 2 (down +
// combine): grid (H/8, tokens), one wave per two experts; each wave
// quantises its two a rows into LDS, does the 8 output rows of w2 of both in
// one MFMA per K-block, and the workgroup sums the k partials in order.
// moe_router_fp8_moe_forward puts the router's logits launch in front and
// lets kernel 1's waves take the top-k of the logits themselves instead of
// reading ids (gateup_gemv_kernel's TOPK).
#include "common.hpp"
#include "gemv.hpp"
#include "grouped.hpp"
#include "route.hpp"
#include "shared.hpp"

#include <mutex>

namespace moe {

constexpr int kMaxHidden = kGemvMaxHidden;
constexpr int kMaxInter = kGemvMaxInter;
constexpr int kMaxK = kGemvMaxTopK;

// Phase marks of the two decode launches, in a separate build of this file
// only (MOE_PHASE_MARKS: libmoeoffload_marks.so, read by the bench's GEMV
// phase probe).  Lane 0 of every wave of the first kMarkWgs workgroups
// records the 100 MHz constant clock (s_memrealtime) at fixed points of its
// kernel, kept in registers and stored at the end with vector stores; each
// call overwrites them, so they hold the last call's.  The marks cost time
// themselves (their clock reads share the scalar/LDS wait counter), so the
// probe reports the marked build's call time beside the plain one.  In the
// product build every PHASE_* macro is empty.
#if defined(MOE_PHASE_MARKS)
constexpr int kMarkWgs = 256, kMarkWaves = 4, kMarks = 8;
__device__ uint64_t g_phase_marks[2 * kMarkWgs * kMarkWaves * kMarks];
__device__ __forceinline__ void phase_marks_store(int kern, const uint64_t* m, int n) {
  const int b = blockIdx.y * gridDim.x + blockIdx.x;
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0 && b < kMarkWgs && wave < kMarkWaves) {
    uint64_t* dst = g_phase_marks + ((kern * kMarkWgs + b) * kMarkWaves + wave) * kMarks;
    for (int i = 0; i < n; ++i) dst[i] = m[i];
  }
}
#define PHASE_MARKS_DECL uint64_t phase_marks_[kMarks]
#define PHASE_MARK(i)                                          \
  do {                                                         \
    __builtin_amdgcn_sched_barrier(0);                         \
    phase_marks_[i] = __builtin_amdgcn_s_memrealtime();        \
    __builtin_amdgcn_sched_barrier(0);                         \
  } while (0)
#define PHASE_MARKS_STORE(kern, n) phase_marks_store(kern, phase_marks_, n)
#else
#define PHASE_MARKS_DECL do {} while (0)
#define PHASE_MARK(i) do {} while (0)
#define PHASE_MARKS_STORE(kern, n) do {} while (0)
#endif

// The id and the routing weight of pair p are read without a branch on
// their dtype: a load inside a branch is waited for inside it, and that wait
// (vmcnt counts in issue order) would also cover every load issued before,
// putting a memory round trip in front of the weight loads.  Both words are
// always read (the same one twice for 32-bit ids, both halves of a float
// weight) and the dtype only selects how they combine.  With p uniform the
// id reads are scalar loads.
//
// The compiler turns a select between a loaded word and another value into
// a branch that loads the word on one side only, and waits for the first
// word inside the other; a second id's loads then go out one round trip
// later.  So the words are loaded first (load_id_words), every id's words
// are pinned together by one empty asm that takes them all (the loads go
// out back to back and are waited for once, where the asm stands), and
// only then combined (id_of).
struct IdWords {
  uint32_t lo, hi;
};
__device__ __forceinline__ IdWords load_id_words(const void* ids, int ids64, int p) {
  const uint32_t* w = static_cast<const uint32_t*>(ids);
  const int i = ids64 ? 2 * p : p;
  return {w[i], w[ids64 ? i + 1 : i]};
}
__device__ __forceinline__ int64_t id_of(IdWords v, int ids64) {
  return ids64 ? static_cast<int64_t>((static_cast<uint64_t>(v.hi) << 32) | v.lo)
               : static_cast<int64_t>(static_cast<int32_t>(v.lo));
}

// Routing weight of pair p as two 16-bit halves (a bf16 weight: the same
// half twice); route_weight() combines them where the value is used.
struct RouteHalves {
  uint32_t lo, hi;
};
__device__ __forceinline__ RouteHalves load_route_halves(const void* w, int wbf16, int p) {
  const uint16_t* w16 = static_cast<const uint16_t*>(w);
  const int i = wbf16 ? p : 2 * p;
  return {w16[i], w16[wbf16 ? i : i + 1]};
}
__device__ __forceinline__ float route_weight(RouteHalves r, int wbf16) {
  return __uint_as_float(wbf16 ? r.lo << 16 : (r.lo | (r.hi << 16)));
}

// ------------------------------------------------------------ kernel 1

// Two 16-row tiles of one (token, expert) pair per workgroup, each split
// over K between kGateUpSplit waves (contiguous ranges of K-blocks).  Every
// wave first issues the loads of its part of the tile (up to kGateUpChunk
// K-blocks of 32 bytes per lane in flight), then the workgroup's waves
// quantise x[t] into LDS together while the weights travel, then each runs
// its MFMAs.  The wave with the first range owns the row sums: it
// accumulates its K-blocks in order and then continues the same chain with
// the block products the other waves left in LDS, so every row is the one
// in-order sum over all K-blocks that the grouped kernel forms
// (bit-identical outputs).
//
// A launch of this kernel is one pass: every wave issues its loads once, and
// its time is the memory time plus each wave's serial instruction stream
// (issue slots, MFMA and LDS latencies), which the loads do not hide.
// Splitting K halves that stream and puts a wave on each of the chip's
// 1024 SIMDs at 8 experts, 2I 1024.  Measured on MI355X (8 experts, H 2048,
// I 512, rocprofv3 kernel durations): 6.5-6.7 us per launch against
// 7.4-7.5 with one wave per tile and 8.9-9.1 with K split four ways;
// reading all of a chunk's B operands before its MFMAs gained nothing
// (the weights' arrival, not the MFMA chain, paces the loop).
constexpr int kGateUpTiles = 2;                  // 16-row tiles per workgroup
constexpr int kGateUpSplit = 2;                  // waves per tile
constexpr int kGateUpWaves = kGateUpSplit * kGateUpTiles;
static_assert(kGateUpTiles == 2, "a workgroup pairs one gate tile with the up tile of its columns");
constexpr int kGateUpChunk = 8;                  // K-blocks in flight per lane

//
// TOPK > 0 (moe_router_fp8_moe_forward): no ids are read; every wave takes
// the top-k of its token's logits itself (TOPK logits per lane, the
// router's wave_topk_keys, so the same picks and weights), its workgroup's
// pick k being lane k's, and workgroup (0, t * top_k) writes token t's ids
// (int32, to `ids`) and routing weights (float32, to `wout`) for the down
// launch.
// The logits' round trip and the top-k take the place of the id load ahead
// of the weight loads, and the top-k needs no launch of its own.
template <bool SHARED, int TOPK>
__global__ __launch_bounds__(64 * kGateUpWaves) void gateup_gemv_kernel(
    const uint16_t* __restrict__ x, const void* __restrict__ ids, int ids64, int32_t top_k,
    const uint8_t* __restrict__ w13, const float* __restrict__ s13, int64_t w13_es,
    int64_t s13_es, int tiled, int32_t n_experts, int32_t hidden, int32_t inter,
    float* __restrict__ act, int32_t tokens, SharedRefs sh, const float* __restrict__ logits,
    float* __restrict__ wout) {
  __shared__ __align__(16) uint8_t xq[kMaxHidden];
  __shared__ float xs[kMaxHidden / 128];
  __shared__ __align__(16) float dpart[kGateUpTiles][kMaxHidden / 128][16];
  __shared__ float spart[kGateUpTiles][kMaxHidden / 128];
  __shared__ __align__(16) float upsum[16];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  if (SHARED && blockIdx.y >= static_cast<unsigned>(tokens * top_k)) {
    // shared expert rows j0, j0 + 1 (gate and up each; j == Is is the sigmoid gate row)
    const int j0 =
        (((blockIdx.y - tokens * top_k) * gridDim.x + blockIdx.x) * kGateUpWaves + wave) *
        kSharedJPW;
    if (j0 > sh.inter) return;                   // the whole wave (no barrier on this branch)
    const uint16_t* rows[2 * kSharedJPW];
#pragma unroll
    for (int i = 0; i < kSharedJPW; ++i) {
      const int j = min(j0 + i, sh.inter);
      const bool gate_row = j == sh.inter;
      rows[2 * i] = gate_row ? sh.wsg : sh.wg + static_cast<int64_t>(j) * hidden;
      rows[2 * i + 1] = gate_row ? sh.wsg : sh.wu + static_cast<int64_t>(j) * hidden;
    }
    for (int t = 0; t < tokens; ++t) {
      float acc[2 * kSharedJPW][1];
      rows_dot_bf16<2 * kSharedJPW, 1, 4>(rows, x, hidden, t, tokens, hidden >> 3, lane, acc);
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < kSharedJPW; ++i) {
          const int j = j0 + i;
          if (j < sh.inter)
            sh.act[static_cast<int64_t>(t) * sh.inter + j] = shared_act(acc[2 * i][0],
                                                                        acc[2 * i + 1][0]);
          else if (j == sh.inter)
            sh.sig[t] = shared_sig(acc[2 * i][0]);
        }
      }
    }
    return;
  }
  // Every workgroup runs this prologue once, and all of it sits on the
  // critical path of a launch whose loads all go out at once: 32-bit
  // arithmetic only (a 64-bit division is ~130 scalar instructions), and
  // x[t], which does not depend on the expert, goes out before the id.
  PHASE_MARKS_DECL;
  PHASE_MARK(0);                       // start
  const int p = blockIdx.y;
  const int t = static_cast<int>(static_cast<uint32_t>(p) / static_cast<uint32_t>(top_k));
  // This wave's first 512 values of x[t] are loaded before the weights:
  // loads retire in issue order (vmcnt), so x issued first can be quantised
  // while the weight tile is still in flight.  No load sits under a branch
  // (lanes and blocks past the end re-read an in-bounds address and ignore
  // it): a conditional load makes the compiler's wait at the join cover
  // every load issued before it, weights included.
  IdWords iw = {0u, 0u};
  if constexpr (TOPK == 0) iw = load_id_words(ids, ids64, p);
  __builtin_amdgcn_sched_barrier(0);
  const uint16_t* xr = x + static_cast<int64_t>(t) * hidden;
  const int i0 = wave * 512 + lane * 8;
  const uint4 xraw = *reinterpret_cast<const uint4*>(xr + (i0 < hidden ? i0 : 0));
  int64_t e;
  if constexpr (TOPK > 0) {
    const int k = p - t * top_k;
    float lv[TOPK];
    load_logits<TOPK>(logits + static_cast<int64_t>(t) * n_experts, n_experts, lv);
    const uint64_t pick = wave_topk_keys<TOPK>(lv, n_experts, top_k);
    const int32_t id = topk_id(pick, top_k);
    e = __builtin_amdgcn_readlane(id, k);
    if (blockIdx.x == 0 && k == 0 && wave == 0) {   // uniform: the weights only here
      const float wt = topk_weight(pick, top_k);
      if (lane < top_k) {
        static_cast<int32_t*>(const_cast<void*>(ids))[p + lane] = id;
        wout[p + lane] = wt;
      }
    }
  } else {
    asm volatile("" : "+s"(iw.lo), "+s"(iw.hi));
    e = id_of(iw, ids64);
  }
  const bool valid = e >= 0 && e < n_experts;
  const int G = hidden >> 7;
  // wave is uniform: so are the tile, the K range and the scale row, which
  // is read with scalar loads
  const int wu = __builtin_amdgcn_readfirstlane(wave);
  const int tile = wu / kGateUpSplit;
  const int part = wu % kGateUpSplit;
  const bool owner = part == 0;          // the wave that forms the row sums
  const int Gs = (G + kGateUpSplit - 1) / kGateUpSplit;   // K-blocks per part
  const int gb = min(part * Gs, G);      // this wave's first K-block
  const int gn = min(gb + Gs, G) - gb;   // and its count (0 for a part past the end)
  // tile 0: gate rows j0..j0+15; tile 1: the up rows of the same columns
  const int j0 = blockIdx.x * 16;
  const int r0 = tile * inter + j0;
  const int q = lane >> 4;
  const OperandWalk ow = operand_walk(r0 + (lane & 15), q, hidden, tiled);
  const uint8_t* wrow = w13 + (valid ? e : 0) * w13_es + ow.off;
  // the tile's block scales go out before the weights (loaded after them,
  // they would add a round trip between the weights' arrival and the MFMAs)
  const float* srow =
      s13 + (valid ? e : 0) * s13_es + static_cast<int64_t>(r0 >> 7) * G;
  float sw[kGateUpChunk];
#pragma unroll
  for (int c = 0; c < kGateUpChunk; ++c) sw[c] = srow[min(gb + c, G - 1)];
  __builtin_amdgcn_sched_barrier(0);
  PHASE_MARK(1);                       // the id is in: the weight loads go out
  v8i a[kGateUpChunk];
#pragma unroll
  for (int c = 0; c < kGateUpChunk; ++c)
    a[c] = load_op_nt(wrow + min(gb + c, G - 1) * ow.kstep, ow.half);
  __builtin_amdgcn_sched_barrier(0);   // every load above is issued before the math below
  // x[t] -> e4m3 codes + per-128 scales in LDS: 8 values per lane, 16 lanes
  // per group, the workgroup's waves taking 512-value slices in turn
  quantize_x8(xraw, i0 < hidden, i0, xq, xs);
  for (int base = (wave + kGateUpWaves) * 512; base < hidden; base += kGateUpWaves * 512) {
    const int i = base + lane * 8;
    const uint4 raw = *reinterpret_cast<const uint4*>(xr + (i < hidden ? i : 0));
    quantize_x8(raw, i < hidden, i, xq, xs);
  }
  PHASE_MARK(2);                       // this wave's share of x quantised
  __syncthreads();
  PHASE_MARK(3);
  float* ap = act + static_cast<int64_t>(p) * inter;
  if (!valid) {   // no such expert (the whole workgroup): poison the columns, read nothing
    if (wu == 0 && lane < 16) ap[j0 + lane] = __builtin_nanf("");
    return;
  }
  // The block product d of K-block g (z = 0) times its scale product sc.
  // The owner folds each into its row sums in order; the other waves
  // leave them in LDS (lane l holds rows 4(l/16)..+3, as every lane with
  // the same l/16 does).
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < gn; k0 += kGateUpChunk) {
    if (k0 > 0) {
#pragma unroll
      for (int c = 0; c < kGateUpChunk; ++c)
        if (k0 + c < gn) {
          a[c] = load_op_nt(wrow + (gb + k0 + c) * ow.kstep, ow.half);
          sw[c] = srow[gb + k0 + c];
        }
    }
    if (!owner) {
#pragma unroll
      for (int c = 0; c < kGateUpChunk; ++c) {
        const int k = k0 + c;
        if (k < gn) {
          const int g = gb + k;
          const v8i b = load_op32(xq + g * 128 + q * 32);
          const v4f z = {0.f, 0.f, 0.f, 0.f};
          const v4f d = mfma_e4m3_16x16x128(a[c], b, z);
          // Every lane stores: the 16 lanes of a row group hold the same
          // four values (B's columns are all x), and a store under a lane
          // condition would let the compiler sink the MFMA into it, where
          // it would run under a partial exec mask.
          *reinterpret_cast<float4*>(&dpart[tile][g][4 * q]) = make_float4(d[0], d[1], d[2], d[3]);
          spart[tile][g] = sw[c] * xs[g];
        }
      }
    } else {
#pragma unroll
      for (int c = 0; c < kGateUpChunk; ++c) {
        const int k = k0 + c;
        if (k < gn) {
          const int g = gb + k;
          const v8i b = load_op32(xq + g * 128 + q * 32);
          const v4f z = {0.f, 0.f, 0.f, 0.f};
          const v4f d = mfma_e4m3_16x16x128(a[c], b, z);
          block_fma(acc, d, sw[c] * xs[g]);
        }
      }
    }
  }
  PHASE_MARK(4);                       // weights in, this wave's MFMAs done
  __syncthreads();
  PHASE_MARK(5);
  if (owner) {
    // unrolled so that the LDS reads of several blocks are in flight at once
#pragma unroll 8
    for (int g = gn; g < G; ++g) {
      const float4 d = *reinterpret_cast<const float4*>(&dpart[tile][g][4 * q]);
      const v4f dv = {d.x, d.y, d.z, d.w};
      block_fma(acc, dv, spart[tile][g]);
    }
    // the up tile's owner hands its row sums over; every lane of a row
    // group stores its (identical) four values
    if (tile == 1)
      *reinterpret_cast<float4*>(&upsum[4 * q]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  }
  __syncthreads();
  if (owner && tile == 0 && (lane & 15) == 0) {
    // a = SiLU(gate) * up of columns j0 + 4q .. +3, as the grouped path's
    // SiLU kernel computes it from the same row sums
    const float4 u = *reinterpret_cast<const float4*>(&upsum[4 * q]);
    *reinterpret_cast<float4*>(ap + j0 + 4 * q) =
        make_float4(silu_mul(acc[0], u.x), silu_mul(acc[1], u.y), silu_mul(acc[2], u.z),
                    silu_mul(acc[3], u.w));
  }
  PHASE_MARK(6);                       // end (SiLU(gate) * up stored)
  PHASE_MARKS_STORE(0, 7);
}

// ------------------------------------------------------------ kernel 2

// Workgroup = 8 output rows, all top_k experts of one token; wave w takes
// experts k = 2w and 2w + 1.  One MFMA holds both: A rows 0-7 are expert
// 2w's 8 rows of w2, rows 8-15 expert 2w+1's, and B columns 0-7 / 8-15 are
// the two experts' quantised activations, so D[r][c] for r, c in the same
// half is the product wanted (the other quadrants are discarded).  The
// weight loads go out first; each wave quantises SiLU(gate)*up of its two
// pairs into LDS while they travel; the k partial results are summed in k
// order.
//
// The grid is H/8 workgroups of ceil(K/2) waves rather than H/16 of K
// waves: the same bytes with the same number of waves, spread over twice as
// many CUs.  Measured on MI355X (8 experts, H 2048, I 512): a read-only
// kernel of each shape took 3.1 against 4.2 us per launch; this kernel
// takes 4.6 us, the 16-row form 5.3-5.6 (both with SiLU on the hardware
// exp2 and reciprocal).  SiLU and the quantisation of the two pairs are
// this kernel's critical path after the loads: with the library SiLU it
// took 5.3-5.4 us, and 4.9 with both replaced by a plain byte copy.
constexpr int kDownChunk = 4;   // K-blocks of w2 in flight per lane (inter 512 = one chunk)
constexpr int kDownRows = 8;    // output rows per workgroup

// The down launch's extra workgroup: the staged table copied into the table.
__device__ __forceinline__ void commit_table(const TableCommit& cm) {
  const int n = static_cast<int>(blockDim.x);
  for (int i = threadIdx.x; i < cm.n_experts; i += n) cm.so_dst[i] = cm.so_src[i];
  for (int i = threadIdx.x; i < cm.cap; i += n) {
    cm.se_dst[i] = cm.se_src[i];
    cm.st_dst[i] = cm.st_src[i];
  }
  if (threadIdx.x == 0) *cm.step_dst = *cm.step_src;
}

template <bool SHARED>
__global__ __launch_bounds__(64 * (kMaxK / 2 + 1)) void down_gemv_kernel(
    const float* __restrict__ act, const void* __restrict__ ids, int ids64,
    const void* __restrict__ weights, int wbf16, int32_t top_k, const uint8_t* __restrict__ w2,
    const float* __restrict__ s2, int64_t w2_es, int64_t s2_es, int tiled, int32_t n_experts,
    int32_t hidden, int32_t inter, const uint16_t* __restrict__ residual,
    uint16_t* __restrict__ out, SharedRefs sh, TableCommit cm) {
  if (static_cast<int>(blockIdx.x) * kDownRows >= hidden) {
    // the workgroup past the output rows (a launch with a staged table)
    if (blockIdx.y == 0) commit_table(cm);
    return;
  }
  __shared__ __align__(16) uint8_t aq[kMaxK][kMaxInter];
  __shared__ float as_[kMaxK][kMaxInter / 128];
  __shared__ __align__(16) float part[kMaxK + 1][kDownRows];   // [kMaxK]: discarded quadrants
  __shared__ float wpart[kMaxK];
  __shared__ float spart[SHARED ? kDownRows : 1];
  PHASE_MARKS_DECL;
  PHASE_MARK(0);                       // start
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.y;
  const int c0 = blockIdx.x * kDownRows;
  const int kwaves = (top_k + 1) >> 1;
  if (SHARED && wave == kwaves) {
    // the shared expert's 8 down rows of this workgroup, token t
    const uint16_t* rows[kDownRows];
#pragma unroll
    for (int i = 0; i < kDownRows; ++i) rows[i] = sh.wd + static_cast<int64_t>(c0 + i) * sh.inter;
    float acc[kDownRows][1];
    rows_dot_bf16<kDownRows, 1, 1>(rows, sh.act, sh.inter, t, t + 1, sh.inter >> 3, lane, acc);
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < kDownRows; ++i) spart[i] = acc[i][0];
    }
    __syncthreads();   // pairs with the routed waves' barrier: threads 0..7 then
    return;            // combine, spart included
  }
  const int wu = __builtin_amdgcn_readfirstlane(wave);
  const int q = lane >> 4;
  // This lane's A row (lane % 16) and B column (lane % 16) belong to the
  // wave's expert slot `half`; its D rows (4q..4q+3) to slot q / 2.
  const int half = (lane & 15) >> 3;
  const int dhalf = q >> 1;
  // the wave's two pairs (uniform); a slot past top_k (odd top_k) repeats
  // pair 2w and is never folded in
  const int k0 = 2 * wu;
  const int k1 = min(2 * wu + 1, top_k - 1);
  const int p0 = t * top_k + k0;
  const int p1 = t * top_k + k1;
  // Both pairs' first 512 activations are loaded before the weights (loads
  // retire in issue order), so their quantisation runs while the weight
  // tile is in flight; they do not depend on the experts and go out before
  // the ids.
  // No load under a branch, for the reason given in the gate/up kernel.
  const int j0 = lane * 8 < inter ? lane * 8 : 0;
  // The residual element of the output this thread combines (threads
  // 0..kDownRows-1) and the token's shared gate go out first: they do not
  // depend on the sums, and loaded in the combine they would add a memory
  // round trip after it.  Without a residual the load reads the first word
  // of the wave's own activation row (loaded next anyway) and is ignored.
  IdWords iw0 = load_id_words(ids, ids64, p0);
  IdWords iw1 = load_id_words(ids, ids64, p1);
  __builtin_amdgcn_sched_barrier(0);
  const float* ap0 = act + static_cast<int64_t>(p0) * inter;
  const int64_t o_mine =
      static_cast<int64_t>(t) * hidden + c0 + min(static_cast<int>(threadIdx.x), kDownRows - 1);
  const uint16_t res_v =
      *(residual ? residual + o_mine : reinterpret_cast<const uint16_t*>(ap0));
  const float sig_v = SHARED ? sh.sig[t] : 0.0f;
  const float* ap1 = act + static_cast<int64_t>(p1) * inter;
  float4 araw0[2], araw1[2];
  araw0[0] = *reinterpret_cast<const float4*>(ap0 + j0);
  araw0[1] = *reinterpret_cast<const float4*>(ap0 + j0 + 4);
  araw1[0] = *reinterpret_cast<const float4*>(ap1 + j0);
  araw1[1] = *reinterpret_cast<const float4*>(ap1 + j0 + 4);
  // the pairs' routing weights, combined only where they are used
  const RouteHalves wr0 = load_route_halves(weights, wbf16, p0);
  const RouteHalves wr1 = load_route_halves(weights, wbf16, p1);
  asm volatile("" : "+s"(iw0.lo), "+s"(iw0.hi), "+s"(iw1.lo), "+s"(iw1.hi));
  const int64_t e0 = id_of(iw0, ids64);
  const int64_t e1 = id_of(iw1, ids64);
  const bool valid0 = e0 >= 0 && e0 < n_experts;
  const bool valid1 = e1 >= 0 && e1 < n_experts;
  const int Gi = inter >> 7;
  // A operand: this lane's row of its slot's expert
  const int64_t ea = half ? (valid1 ? e1 : 0) : (valid0 ? e0 : 0);
  const OperandWalk ow = operand_walk(c0 + (lane & 7), q, inter, tiled);
  const uint8_t* wrow = w2 + ea * w2_es + ow.off;
  // block scales of the slot that owns this lane's D rows, before the weights
  const int64_t ed = dhalf ? (valid1 ? e1 : 0) : (valid0 ? e0 : 0);
  const float* srow = s2 + ed * s2_es + static_cast<int64_t>(c0 >> 7) * Gi;
  float sw[kDownChunk];
#pragma unroll
  for (int c = 0; c < kDownChunk; ++c) sw[c] = srow[c < Gi ? c : Gi - 1];
  __builtin_amdgcn_sched_barrier(0);
  PHASE_MARK(1);                       // the ids are in: the weight loads go out
  v8i a[kDownChunk];
#pragma unroll
  for (int c = 0; c < kDownChunk; ++c)
    a[c] = load_op_nt(wrow + (c < Gi ? c : Gi - 1) * ow.kstep, ow.half);
  __builtin_amdgcn_sched_barrier(0);   // every load above is issued before the math below
  // both pairs' activations, quantised per 128 into LDS: 16 lanes x 8
  quantize8_f32(araw0, lane * 8 < inter, lane * 8, aq[k0], as_[k0]);
  quantize8_f32(araw1, lane * 8 < inter, lane * 8, aq[k0 + 1], as_[k0 + 1]);
  for (int base = 512; base < inter; base += 512) {
    const int j = base + lane * 8;
    const int jj = j < inter ? j : 0;
    float4 ar[2];
    ar[0] = *reinterpret_cast<const float4*>(ap0 + jj);
    ar[1] = *reinterpret_cast<const float4*>(ap0 + jj + 4);
    quantize8_f32(ar, j < inter, j, aq[k0], as_[k0]);
    ar[0] = *reinterpret_cast<const float4*>(ap1 + jj);
    ar[1] = *reinterpret_cast<const float4*>(ap1 + jj + 4);
    quantize8_f32(ar, j < inter, j, aq[k0 + 1], as_[k0 + 1]);
  }
  // aq[k0..k0+1] and as_[k0..k0+1] are this wave's own: its LDS accesses
  // complete in order, so a wave-scope fence (which keeps the compiler from
  // moving the reads above the writes) replaces a workgroup barrier
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  PHASE_MARK(2);                       // both pairs' activations quantised

  // B operand: this lane's column is its slot's activation; the row sums
  // of slot dhalf run in K-block order with that slot's scales
  const uint8_t* bq = aq[k0 + half];
  const float* asd = as_[k0 + dhalf];
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  for (int g0 = 0; g0 < Gi; g0 += kDownChunk) {
    if (g0 > 0) {
#pragma unroll
      for (int c = 0; c < kDownChunk; ++c)
        if (g0 + c < Gi) {
          a[c] = load_op_nt(wrow + (g0 + c) * ow.kstep, ow.half);
          sw[c] = srow[g0 + c];
        }
    }
#pragma unroll
    for (int c = 0; c < kDownChunk; ++c) {
      const int g = g0 + c;
      if (g < Gi) {
        const v8i b = load_op32(bq + g * 128 + q * 32);
        const v4f z = {0.f, 0.f, 0.f, 0.f};
        const v4f d = mfma_e4m3_16x16x128(a[c], b, z);
        block_fma(acc, d, sw[c] * asd[g]);
      }
    }
  }
  {
    // Every lane stores, unconditionally (a store under a lane condition
    // would let the compiler sink the MFMAs into it, under a partial exec
    // mask): lanes whose column is in their rows' half write the slot's 4
    // rows (the 8 such lanes per row group write the same values), the
    // others write the discard row.
    const int kd = k0 + dhalf;
    const bool mine = half == dhalf;
    const bool ok = dhalf ? valid1 : valid0;
    const float nan = __builtin_nanf("");
    float* dst = mine ? &part[kd][4 * (q & 1)] : &part[kMaxK][4 * (q & 1)];
    *reinterpret_cast<float4*>(dst) =
        ok ? make_float4(acc[0], acc[1], acc[2], acc[3]) : make_float4(nan, nan, nan, nan);
  }
  wpart[k0] = route_weight(wr0, wbf16);
  wpart[k0 + 1] = route_weight(wr1, wbf16);
  PHASE_MARK(3);                       // weights in, MFMAs done, partials stored
  __syncthreads();
  PHASE_MARK(4);
  if (threadIdx.x < kDownRows) {
    // sum = fma(w_k, y_k, sum), k in order: the combine of the grouped path
    // too.  All kMaxK partials are read at once (one LDS round trip); the
    // slots past top_k are never folded in.
    float wk[kMaxK], yk[kMaxK];
#pragma unroll
    for (int k = 0; k < kMaxK; ++k) {
      wk[k] = wpart[k];
      yk[k] = part[k][threadIdx.x];
    }
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kMaxK; ++k)
      if (k < top_k) sum = fmaf(wk[k], yk[k], sum);
    const int64_t o = static_cast<int64_t>(t) * hidden + c0 + threadIdx.x;
    uint16_t y = f32_to_bf16(sum);
    if (SHARED) {
      // out = residual + (routed + sig * shared), as moe_shared_down on the routed output
      y = shared_out(spart[threadIdx.x], sig_v, true, y, residual != nullptr, res_v);
    } else if (residual) {
      y = f32_to_bf16(bf16_to_f32(res_v) + bf16_to_f32(y));
    }
    out[o] = y;
  }
  PHASE_MARK(5);                       // end (outputs stored)
  PHASE_MARKS_STORE(1, 6);
}

// ------------------------------------------------ bf16 activations (mode 3)

// moe_fp8_moe_forward_ex mode 3: the per-pair GEMV with the activations kept
// in bf16 instead of quantised to e4m3, the numerics of the dequantise-then-
// matmul path (bin/offload.py's CPU expert path; the closed form of
// notes/13-non-ada-gpus.md:43-53):
//   h[p][r] = sum_g s13[e][r/128][g] * <w13[e][r][g*128:+128], x[t][g*128:+128]>
//   a = SiLU(h[:I]) * h[I:] in float32, rounded to bf16 for the down products
//   y[c]    = sum_g s2[e][c/128][g] * <w2[e][c][g*128:+128], a[g*128:+128]>
//   out[t]  = fma(w[t][k], y_k, out[t]) for k in order, float32 -> bf16.
// An e4m3 weight converts to bf16 exactly (v_cvt_scalef32_pk_bf16_fp8, scale
// 1), and a bf16 product is exact in float32, so each 128-term block product
// is four v_mfma_f32_16x16x32_bf16 summing exact products in float32.  A
// lane's 32 weight bytes of a K-block hold reduction indices 32q..32q+31
// (q = lane / 16, in either record layout); MFMA j takes indices
// 32q + 8j..+7 from each lane group, and its B operand the activation at
// those indices, so the four MFMAs cover the block once.  Grids, waves, the
// weights' loads, the in-order K-block chains and the k-order combine are
// the e4m3 kernels'.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// 8 e4m3 bytes (two words, lowest byte first) -> 8 bf16 in the same order.
__device__ __forceinline__ bf16x8 e4m3x8_to_bf16(uint32_t lo, uint32_t hi) {
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
  return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// One K-block's product: the lane's 32 weight bytes `a` against the bf16
// activations `b` at the block's indices 32q.. (b points at index 32q).
__device__ __forceinline__ v4f block_bf16(v8i a, const uint16_t* b) {
  v4f d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x8 bj = *reinterpret_cast<const bf16x8*>(b + 8 * j);
    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        e4m3x8_to_bf16(static_cast<uint32_t>(a[2 * j]), static_cast<uint32_t>(a[2 * j + 1])), bj,
        d, 0, 0, 0);
  }
  return d;
}

// Gate/up + SiLU with bf16 activations: gateup_gemv_kernel's grid and waves,
// x[t] copied into LDS as it is instead of quantised.
__global__ __launch_bounds__(64 * kGateUpWaves) void gateup_gemv_a16_kernel(
    const uint16_t* __restrict__ x, const void* __restrict__ ids, int ids64, int32_t top_k,
    const uint8_t* __restrict__ w13, const float* __restrict__ s13, int64_t w13_es,
    int64_t s13_es, int tiled, int32_t n_experts, int32_t hidden, int32_t inter,
    float* __restrict__ act) {
  __shared__ __align__(16) uint16_t xb[kMaxHidden];
  __shared__ __align__(16) float dpart[kGateUpTiles][kMaxHidden / 128][16];
  __shared__ float spart[kGateUpTiles][kMaxHidden / 128];
  __shared__ __align__(16) float upsum[16];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int p = blockIdx.y;
  const int t = static_cast<int>(static_cast<uint32_t>(p) / static_cast<uint32_t>(top_k));
  // the id's words, then this wave's first 512 values of x[t], go out
  // before the weights (the order of gateup_gemv_kernel)
  IdWords iw = load_id_words(ids, ids64, p);
  __builtin_amdgcn_sched_barrier(0);
  const uint16_t* xr = x + static_cast<int64_t>(t) * hidden;
  const int i0 = wave * 512 + lane * 8;
  const uint4 xraw = *reinterpret_cast<const uint4*>(xr + (i0 < hidden ? i0 : 0));
  asm volatile("" : "+s"(iw.lo), "+s"(iw.hi));
  const int64_t e = id_of(iw, ids64);
  const bool valid = e >= 0 && e < n_experts;
  const int G = hidden >> 7;
  const int wu = __builtin_amdgcn_readfirstlane(wave);
  const int tile = wu / kGateUpSplit;
  const int part = wu % kGateUpSplit;
  const bool owner = part == 0;
  const int Gs = (G + kGateUpSplit - 1) / kGateUpSplit;
  const int gb = min(part * Gs, G);
  const int gn = min(gb + Gs, G) - gb;
  const int j0 = blockIdx.x * 16;
  const int r0 = tile * inter + j0;
  const int q = lane >> 4;
  const OperandWalk ow = operand_walk(r0 + (lane & 15), q, hidden, tiled);
  const uint8_t* wrow = w13 + (valid ? e : 0) * w13_es + ow.off;
  const float* srow =
      s13 + (valid ? e : 0) * s13_es + static_cast<int64_t>(r0 >> 7) * G;
  float sw[kGateUpChunk];
#pragma unroll
  for (int c = 0; c < kGateUpChunk; ++c) sw[c] = srow[min(gb + c, G - 1)];
  __builtin_amdgcn_sched_barrier(0);
  v8i a[kGateUpChunk];
#pragma unroll
  for (int c = 0; c < kGateUpChunk; ++c)
    a[c] = load_op_nt(wrow + min(gb + c, G - 1) * ow.kstep, ow.half);
  __builtin_amdgcn_sched_barrier(0);
  if (i0 < hidden) *reinterpret_cast<uint4*>(&xb[i0]) = xraw;
  for (int base = (wave + kGateUpWaves) * 512; base < hidden; base += kGateUpWaves * 512) {
    const int i = base + lane * 8;
    const uint4 raw = *reinterpret_cast<const uint4*>(xr + (i < hidden ? i : 0));
    if (i < hidden) *reinterpret_cast<uint4*>(&xb[i]) = raw;
  }
  __syncthreads();
  float* ap = act + static_cast<int64_t>(p) * inter;
  if (!valid) {
    if (wu == 0 && lane < 16) ap[j0 + lane] = __builtin_nanf("");
    return;
  }
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < gn; k0 += kGateUpChunk) {
    if (k0 > 0) {
#pragma unroll
      for (int c = 0; c < kGateUpChunk; ++c)
        if (k0 + c < gn) {
          a[c] = load_op_nt(wrow + (gb + k0 + c) * ow.kstep, ow.half);
          sw[c] = srow[gb + k0 + c];
        }
    }
#pragma unroll
    for (int c = 0; c < kGateUpChunk; ++c) {
      const int k = k0 + c;
      if (k < gn) {
        const int g = gb + k;
        const v4f d = block_bf16(a[c], xb + g * 128 + q * 32);
        if (owner) {
          block_fma(acc, d, sw[c]);
        } else {
          // every lane stores (see gateup_gemv_kernel)
          *reinterpret_cast<float4*>(&dpart[tile][g][4 * q]) = make_float4(d[0], d[1], d[2], d[3]);
          spart[tile][g] = sw[c];
        }
      }
    }
  }
  __syncthreads();
  if (owner) {
#pragma unroll 8
    for (int g = gn; g < G; ++g) {
      const float4 d = *reinterpret_cast<const float4*>(&dpart[tile][g][4 * q]);
      const v4f dv = {d.x, d.y, d.z, d.w};
      block_fma(acc, dv, spart[tile][g]);
    }
    if (tile == 1)
      *reinterpret_cast<float4*>(&upsum[4 * q]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  }
  __syncthreads();
  if (owner && tile == 0 && (lane & 15) == 0) {
    const float4 u = *reinterpret_cast<const float4*>(&upsum[4 * q]);
    *reinterpret_cast<float4*>(ap + j0 + 4 * q) =
        make_float4(silu_mul(acc[0], u.x), silu_mul(acc[1], u.y), silu_mul(acc[2], u.z),
                    silu_mul(acc[3], u.w));
  }
}

// Down + combine with bf16 activations: down_gemv_kernel's grid and waves,
// each wave rounding its two pairs' SiLU(gate) * up rows to bf16 into LDS
// instead of quantising them.
__global__ __launch_bounds__(64 * (kMaxK / 2)) void down_gemv_a16_kernel(
    const float* __restrict__ act, const void* __restrict__ ids, int ids64,
    const void* __restrict__ weights, int wbf16, int32_t top_k, const uint8_t* __restrict__ w2,
    const float* __restrict__ s2, int64_t w2_es, int64_t s2_es, int tiled, int32_t n_experts,
    int32_t hidden, int32_t inter, const uint16_t* __restrict__ residual,
    uint16_t* __restrict__ out) {
  __shared__ __align__(16) uint16_t ab[kMaxK][kMaxInter];
  __shared__ __align__(16) float part[kMaxK + 1][kDownRows];
  __shared__ float wpart[kMaxK];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.y;
  const int c0 = blockIdx.x * kDownRows;
  const int wu = __builtin_amdgcn_readfirstlane(wave);
  const int q = lane >> 4;
  const int half = (lane & 15) >> 3;
  const int dhalf = q >> 1;
  const int k0 = 2 * wu;
  const int k1 = min(2 * wu + 1, top_k - 1);
  const int p0 = t * top_k + k0;
  const int p1 = t * top_k + k1;
  const int j0 = lane * 8 < inter ? lane * 8 : 0;
  IdWords iw0 = load_id_words(ids, ids64, p0);
  IdWords iw1 = load_id_words(ids, ids64, p1);
  __builtin_amdgcn_sched_barrier(0);
  const float* ap0 = act + static_cast<int64_t>(p0) * inter;
  const int64_t o_mine =
      static_cast<int64_t>(t) * hidden + c0 + min(static_cast<int>(threadIdx.x), kDownRows - 1);
  const uint16_t res_v =
      *(residual ? residual + o_mine : reinterpret_cast<const uint16_t*>(ap0));
  const float* ap1 = act + static_cast<int64_t>(p1) * inter;
  float4 araw0[2], araw1[2];
  araw0[0] = *reinterpret_cast<const float4*>(ap0 + j0);
  araw0[1] = *reinterpret_cast<const float4*>(ap0 + j0 + 4);
  araw1[0] = *reinterpret_cast<const float4*>(ap1 + j0);
  araw1[1] = *reinterpret_cast<const float4*>(ap1 + j0 + 4);
  const RouteHalves wr0 = load_route_halves(weights, wbf16, p0);
  const RouteHalves wr1 = load_route_halves(weights, wbf16, p1);
  asm volatile("" : "+s"(iw0.lo), "+s"(iw0.hi), "+s"(iw1.lo), "+s"(iw1.hi));
  const int64_t e0 = id_of(iw0, ids64);
  const int64_t e1 = id_of(iw1, ids64);
  const bool valid0 = e0 >= 0 && e0 < n_experts;
  const bool valid1 = e1 >= 0 && e1 < n_experts;
  const int Gi = inter >> 7;
  const int64_t ea = half ? (valid1 ? e1 : 0) : (valid0 ? e0 : 0);
  const OperandWalk ow = operand_walk(c0 + (lane & 7), q, inter, tiled);
  const uint8_t* wrow = w2 + ea * w2_es + ow.off;
  const int64_t ed = dhalf ? (valid1 ? e1 : 0) : (valid0 ? e0 : 0);
  const float* srow = s2 + ed * s2_es + static_cast<int64_t>(c0 >> 7) * Gi;
  float sw[kDownChunk];
#pragma unroll
  for (int c = 0; c < kDownChunk; ++c) sw[c] = srow[c < Gi ? c : Gi - 1];
  __builtin_amdgcn_sched_barrier(0);
  v8i a[kDownChunk];
#pragma unroll
  for (int c = 0; c < kDownChunk; ++c)
    a[c] = load_op_nt(wrow + (c < Gi ? c : Gi - 1) * ow.kstep, ow.half);
  __builtin_amdgcn_sched_barrier(0);
  // both pairs' activation rows -> bf16 in LDS, 8 values per lane per 512
  auto put8 = [&](const float4* r, int j, uint16_t* dst) {
    if (j < inter) {
      const uint4 v = {
          static_cast<uint32_t>(f32_to_bf16(r[0].x)) | (static_cast<uint32_t>(f32_to_bf16(r[0].y)) << 16),
          static_cast<uint32_t>(f32_to_bf16(r[0].z)) | (static_cast<uint32_t>(f32_to_bf16(r[0].w)) << 16),
          static_cast<uint32_t>(f32_to_bf16(r[1].x)) | (static_cast<uint32_t>(f32_to_bf16(r[1].y)) << 16),
          static_cast<uint32_t>(f32_to_bf16(r[1].z)) | (static_cast<uint32_t>(f32_to_bf16(r[1].w)) << 16)};
      *reinterpret_cast<uint4*>(dst + j) = v;
    }
  };
  put8(araw0, lane * 8, ab[k0]);
  put8(araw1, lane * 8, ab[k0 + 1]);
  for (int base = 512; base < inter; base += 512) {
    const int j = base + lane * 8;
    const int jj = j < inter ? j : 0;
    float4 ar[2];
    ar[0] = *reinterpret_cast<const float4*>(ap0 + jj);
    ar[1] = *reinterpret_cast<const float4*>(ap0 + jj + 4);
    put8(ar, j, ab[k0]);
    ar[0] = *reinterpret_cast<const float4*>(ap1 + jj);
    ar[1] = *reinterpret_cast<const float4*>(ap1 + jj + 4);
    put8(ar, j, ab[k0 + 1]);
  }
  // the wave's own rows: a wave-scope fence stands for a barrier (see down_gemv_kernel)
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const uint16_t* bq = ab[k0 + half];
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  for (int g0 = 0; g0 < Gi; g0 += kDownChunk) {
    if (g0 > 0) {
#pragma unroll
      for (int c = 0; c < kDownChunk; ++c)
        if (g0 + c < Gi) {
          a[c] = load_op_nt(wrow + (g0 + c) * ow.kstep, ow.half);
          sw[c] = srow[g0 + c];
        }
    }
#pragma unroll
    for (int c = 0; c < kDownChunk; ++c) {
      const int g = g0 + c;
      if (g < Gi) block_fma(acc, block_bf16(a[c], bq + g * 128 + q * 32), sw[c]);
    }
  }
  {
    const int kd = k0 + dhalf;
    const bool mine = half == dhalf;
    const bool ok = dhalf ? valid1 : valid0;
    const float nan = __builtin_nanf("");
    float* dst = mine ? &part[kd][4 * (q & 1)] : &part[kMaxK][4 * (q & 1)];
    *reinterpret_cast<float4*>(dst) =
        ok ? make_float4(acc[0], acc[1], acc[2], acc[3]) : make_float4(nan, nan, nan, nan);
  }
  wpart[k0] = route_weight(wr0, wbf16);
  wpart[k0 + 1] = route_weight(wr1, wbf16);
  __syncthreads();
  if (threadIdx.x < kDownRows) {
    float wk[kMaxK], yk[kMaxK];
#pragma unroll
    for (int k = 0; k < kMaxK; ++k) {
      wk[k] = wpart[k];
      yk[k] = part[k][threadIdx.x];
    }
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kMaxK; ++k)
      if (k < top_k) sum = fmaf(wk[k], yk[k], sum);
    const int64_t o = static_cast<int64_t>(t) * hidden + c0 + threadIdx.x;
    uint16_t y = f32_to_bf16(sum);
    if (residual) y = f32_to_bf16(bf16_to_f32(res_v) + bf16_to_f32(y));
    out[o] = y;
  }
}

// The two decode launches; `sh` (nullable) carries the shared expert along.
// The router of up to 16 tokens in front of the GEMV launches: its logits launch
// (gate weight, bias, logit rounding, the logits buffer), then the top-k
// made inside the gate/up launch (gateup_gemv_kernel's TOPK), which writes
// the ids and weights.
struct RouterTopK {
  const void* w_gate;
  const float* bias;
  int bf16_logits;
  float* logits;
  int32_t* ids;
  float* weights;
};

static int launch_gemv(const uint16_t* x, const void* ids, int ids64, const void* weights,
                       int wbf16, int32_t tokens, int32_t top_k, const uint8_t* w13,
                       const float* s13, const uint8_t* w2, const float* s2,
                       const moe_expert_strides& es, int32_t n_experts, int32_t hidden,
                       int32_t inter, const uint16_t* residual, uint16_t* out, float* h,
                       const SharedRefs* sh, hipStream_t s, const RouterTopK* rt = nullptr) {
  const int64_t pairs = static_cast<int64_t>(tokens) * top_k;
  const unsigned gx = static_cast<unsigned>((2 * inter) / 16);
  if (sh) {
    // extra rows of workgroups for the shared expert's Is + 1 rows (the last: sigmoid gate)
    const unsigned per_y = kSharedJPW * (gx / kGateUpTiles) * kGateUpWaves;
    const unsigned sy = static_cast<unsigned>((sh->inter + 1 + per_y - 1) / per_y);
    hipLaunchKernelGGL((gateup_gemv_kernel<true, 0>), dim3(gx / kGateUpTiles, pairs + sy),
                       dim3(64 * kGateUpWaves), 0, s, x, ids,
                       ids64, top_k, w13, s13, es.w13, es.s13, static_cast<int>(es.layout),
                       n_experts, hidden, inter, h, tokens, *sh, nullptr, nullptr);
  } else if (rt) {
    // one token: the ids and weights the down launch reads are the top-k's
    ids = rt->ids;
    ids64 = 0;
    weights = rt->weights;
    wbf16 = 0;
    if (n_experts <= 256)
      hipLaunchKernelGGL((gateup_gemv_kernel<false, 4>), dim3(gx / kGateUpTiles, pairs),
                         dim3(64 * kGateUpWaves), 0, s, x, ids, 0, top_k, w13, s13, es.w13,
                         es.s13, static_cast<int>(es.layout), n_experts, hidden, inter, h, tokens,
                         SharedRefs{}, rt->logits, rt->weights);
    else
      hipLaunchKernelGGL((gateup_gemv_kernel<false, 16>), dim3(gx / kGateUpTiles, pairs),
                         dim3(64 * kGateUpWaves), 0, s, x, ids, 0, top_k, w13, s13, es.w13,
                         es.s13, static_cast<int>(es.layout), n_experts, hidden, inter, h, tokens,
                         SharedRefs{}, rt->logits, rt->weights);
  } else {
    hipLaunchKernelGGL((gateup_gemv_kernel<false, 0>), dim3(gx / kGateUpTiles, pairs),
                       dim3(64 * kGateUpWaves), 0, s, x, ids, ids64,
                       top_k, w13, s13, es.w13, es.s13, static_cast<int>(es.layout), n_experts,
                       hidden, inter, h, tokens, SharedRefs{}, nullptr, nullptr);
  }
  int rc = check_launch("moe_fp8_moe_forward(gate/up)");
  if (rc) return rc;
  if (sh) {
    hipLaunchKernelGGL(down_gemv_kernel<true>, dim3(hidden / kDownRows, tokens),
                       dim3(64 * ((top_k + 1) / 2 + 1)),
                       0, s, h, ids, ids64, weights, wbf16, top_k, w2, s2, es.w2, es.s2,
                       static_cast<int>(es.layout), n_experts, hidden, inter, residual, out, *sh,
                       TableCommit{});
  } else {
    hipLaunchKernelGGL(down_gemv_kernel<false>, dim3(hidden / kDownRows, tokens),
                       dim3(64 * ((top_k + 1) / 2)), 0, s,
                       h, ids, ids64, weights, wbf16, top_k, w2, s2, es.w2, es.s2,
                       static_cast<int>(es.layout), n_experts, hidden, inter, residual, out,
                       SharedRefs{}, TableCommit{});
  }
  return check_launch("moe_fp8_moe_forward(down)");
}

// The two decode launches of mode 3 (bf16 activations).
static int launch_gemv_a16(const uint16_t* x, const void* ids, int ids64, const void* weights,
                           int wbf16, int32_t tokens, int32_t top_k, const uint8_t* w13,
                           const float* s13, const uint8_t* w2, const float* s2,
                           const moe_expert_strides& es, int32_t n_experts, int32_t hidden,
                           int32_t inter, const uint16_t* residual, uint16_t* out, float* h,
                           hipStream_t s) {
  const int64_t pairs = static_cast<int64_t>(tokens) * top_k;
  const unsigned gx = static_cast<unsigned>((2 * inter) / 16);
  hipLaunchKernelGGL(gateup_gemv_a16_kernel, dim3(gx / kGateUpTiles, pairs),
                     dim3(64 * kGateUpWaves), 0, s, x, ids, ids64, top_k, w13, s13, es.w13,
                     es.s13, static_cast<int>(es.layout), n_experts, hidden, inter, h);
  int rc = check_launch("moe_fp8_moe_forward(gate/up, bf16 activations)");
  if (rc) return rc;
  hipLaunchKernelGGL(down_gemv_a16_kernel, dim3(hidden / kDownRows, tokens),
                     dim3(64 * ((top_k + 1) / 2)), 0, s, h, ids, ids64, weights, wbf16, top_k, w2,
                     s2, es.w2, es.s2, static_cast<int>(es.layout), n_experts, hidden, inter,
                     residual, out);
  return check_launch("moe_fp8_moe_forward(down, bf16 activations)");
}

int launch_down_gemv(const float* act, const int32_t* slots, const void* weights, int wbf16,
                     int32_t tokens, int32_t top_k, const uint8_t* w2, const float* s2,
                     int64_t w2_es, int64_t s2_es, int tiled, int32_t n_slots, int32_t hidden,
                     int32_t inter, const uint16_t* residual, uint16_t* out,
                     const SharedRefs* sh, hipStream_t s, const TableCommit* commit) {
  const TableCommit cm = commit ? *commit : TableCommit{};
  const unsigned extra = commit ? 1u : 0u;
  if (sh) {
    hipLaunchKernelGGL(down_gemv_kernel<true>, dim3(hidden / kDownRows + extra, tokens),
                       dim3(64 * ((top_k + 1) / 2 + 1)), 0, s, act, slots, 0, weights, wbf16,
                       top_k, w2, s2, w2_es, s2_es, tiled, n_slots, hidden, inter, residual, out,
                       *sh, cm);
  } else {
    hipLaunchKernelGGL(down_gemv_kernel<false>, dim3(hidden / kDownRows + extra, tokens),
                       dim3(64 * ((top_k + 1) / 2)), 0, s, act, slots, 0, weights, wbf16, top_k,
                       w2, s2, w2_es, s2_es, tiled, n_slots, hidden, inter, residual, out,
                       SharedRefs{}, cm);
  }
  return check_launch("down_gemv_kernel");
}

}  // namespace moe

using namespace moe;

// Calls of at most this many tokens take the per-pair GEMV kernels by default;
// larger ones the grouped kernels, which read each expert's weights once.
// Measured on MI355X (top-8 of 256 uniform, H 2048, I 512, tile-ordered
// records rotating over 2048 of them, graph of back-to-back calls): GEMV
// 9.7 / 20.9 / 37.3 / 68.7 us against grouped 47.4 / 56.1 / 54.8 / 68.7 us
// at 1 / 4 / 8 / 16 tokens, and 82.4 against 77.5 us at 20: the GEMV's
// re-read of shared experts costs less than the grouped path's four
// launches up to 16 tokens.
constexpr int32_t kGemvMaxTokens = 16;
// The block call carries the shared expert in the GEMV launches up to this
// many tokens (its gate/up workgroups take the tokens one after another);
// beyond, the routed call is followed by the two shared-expert kernels.
constexpr int32_t kCarrySharedMaxTokens = 2;

static bool use_grouped(int32_t tokens, int32_t hidden, int32_t mode) {
  if (mode == 1 || mode == 3) return false;
  if (mode == 2) return true;
  return tokens > kGemvMaxTokens;
}

extern "C" size_t moe_fp8_moe_workspace(int32_t tokens, int32_t top_k, int32_t n_experts,
                                        int32_t hidden, int32_t inter) {
  if (tokens <= 0 || top_k <= 0 || inter <= 0 || hidden <= 0 || n_experts <= 0) return 256;
  // per-pair GEMV: one float32 row of 2*inter per (token, expert) pair
  const size_t h = static_cast<size_t>(tokens) * top_k * 2 * inter * sizeof(float);
  size_t need = (h + 255) & ~static_cast<size_t>(255);
  // grouped: permutation, quantised activations and permuted outputs
  const size_t g = grouped_layout(tokens, top_k, n_experts, hidden, inter).total;
  return need > g ? need : g;
}

// ---------------------------------------------------------------------------
// The allocation-free forward: moe_fp8_moe_forward_ex with its workspace in
// a file-scope device array instead of a caller's buffer.
//
// Each GPU the library runs on holds its own copy of `scratch` until the
// process ends.  In host code the name `scratch` is only a stand-in for the
// variable, not a device address: the address each device's copy has is
// looked up with hipGetSymbolAddress, once per device with that device
// current, and only that address ever reaches a kernel.  Every call on one
// GPU uses the same copy, so calls that overlap on one GPU (two streams, two
// threads) race on it.  No kernel of the forward reads a workspace byte it
// has not written earlier in the same call, so nothing is cleared between
// calls.

static size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

constexpr size_t kNoAllocScratchBytes = MOE_NOALLOC_SCRATCH_BYTES;
static_assert(kNoAllocScratchBytes % 256 == 0, "scratch size must keep 256-byte alignment");
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_dev[kMaxDevices];

// This device's copy of `scratch`, looked up on the first call on it.
static int scratch_address(hipStream_t s, void** addr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("moe_fp8_moe_forward_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return static_cast<int>(e);
  }
  MOE_REQUIRE(dev >= 0 && dev < kMaxDevices,
              "moe_fp8_moe_forward_noalloc: device %d beyond the %d this library tracks", dev,
              kMaxDevices);
  if (s != nullptr) {
    // the address is per device: a stream of another device would get the
    // current device's copy
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(s, &sdev);
    if (e != hipSuccess) {
      set_error("moe_fp8_moe_forward_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    MOE_REQUIRE(static_cast<int>(sdev) == dev,
                "moe_fp8_moe_forward_noalloc: the stream belongs to device %d, the current "
                "device is %d", static_cast<int>(sdev), dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("moe_fp8_moe_forward_noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                dev, hipGetErrorString(e));
      return e != hipSuccess ? static_cast<int>(e) : MOE_EINVAL;
    }
    g_scratch_dev[dev] = p;
  }
  *addr = g_scratch_dev[dev];
  return MOE_OK;
}

// The routed-expert call: preconditions, then the GEMV or grouped path.
// `sh` (nullable) asks for the shared expert on the GEMV path; *fused tells
// whether it was carried along (the caller runs it after a grouped call).
static int forward_impl(const void* x, const void* ids, int32_t ids_dtype, const void* weights,
                        int32_t w_dtype, int32_t tokens, int32_t top_k, const void* w13,
                        const float* s13, const void* w2, const float* s2, int32_t n_experts,
                        int32_t hidden, int32_t inter, const moe_expert_strides* strides,
                        const void* residual, void* out, void* workspace, size_t workspace_bytes,
                        int32_t mode, const SharedRefs* sh, bool* fused, void* stream,
                        bool static_scratch = false, const RouterTopK* rt = nullptr) {
  *fused = false;
  MOE_REQUIRE(tokens >= 0, "moe_fp8_moe_forward: tokens < 0");
  MOE_REQUIRE(top_k >= 1 && top_k <= kMaxK, "moe_fp8_moe_forward: need 1 <= top_k <= %d", kMaxK);
  MOE_REQUIRE(hidden >= 128 && hidden % 128 == 0 && hidden <= kMaxHidden,
              "moe_fp8_moe_forward: hidden must be a multiple of 128 in [128, %d] (got %d)",
              kMaxHidden, hidden);
  MOE_REQUIRE(inter >= 128 && inter % 128 == 0 && inter <= kMaxInter,
              "moe_fp8_moe_forward: inter must be a multiple of 128 in [128, %d] (got %d)",
              kMaxInter, inter);
  MOE_REQUIRE(n_experts >= 1, "moe_fp8_moe_forward: n_experts < 1");
  MOE_REQUIRE(ids_dtype == MOE_I32 || ids_dtype == MOE_I64, "moe_fp8_moe_forward: bad ids_dtype");
  MOE_REQUIRE(w_dtype == MOE_F32 || w_dtype == MOE_BF16, "moe_fp8_moe_forward: bad w_dtype");
  MOE_REQUIRE(mode >= 0 && mode <= 3, "moe_fp8_moe_forward: mode must be 0, 1, 2 or 3");
  if (tokens == 0) return MOE_OK;   // an empty call touches nothing (its tensors may be NULL)
  MOE_REQUIRE(x && ids && weights && w13 && s13 && w2 && s2 && out,
              "moe_fp8_moe_forward: NULL pointer");
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w13) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(w2) % 16 == 0,
              "moe_fp8_moe_forward: x, w13 and w2 must be 16-byte aligned");
  moe_expert_strides es;
  if (strides) {
    es = *strides;
  } else {
    es.w13 = 2LL * inter * hidden;
    es.s13 = (2LL * inter / 128) * (hidden / 128);
    es.w2 = static_cast<int64_t>(hidden) * inter;
    es.s2 = (static_cast<int64_t>(hidden) / 128) * (inter / 128);
    es.layout = MOE_LAYOUT_ROWS;
  }
  MOE_REQUIRE(es.layout == MOE_LAYOUT_ROWS || es.layout == MOE_LAYOUT_TILES,
              "moe_fp8_moe_forward: strides->layout must be MOE_LAYOUT_ROWS or MOE_LAYOUT_TILES");
  MOE_REQUIRE(es.w13 >= 2LL * inter * hidden && es.w2 >= static_cast<int64_t>(hidden) * inter &&
                  es.s13 >= (2LL * inter / 128) * (hidden / 128) &&
                  es.s2 >= (static_cast<int64_t>(hidden) / 128) * (inter / 128),
              "moe_fp8_moe_forward: expert strides smaller than one expert");
  MOE_REQUIRE(es.w13 % 16 == 0 && es.w2 % 16 == 0,
              "moe_fp8_moe_forward: w13/w2 expert strides must be multiples of 16 bytes");
  const size_t need = moe_fp8_moe_workspace(tokens, top_k, n_experts, hidden, inter);
  if (static_scratch) {
    // moe_fp8_moe_forward_noalloc: the library's per-GPU array is the workspace
    MOE_REQUIRE(need <= kNoAllocScratchBytes,
                "moe_fp8_moe_forward_noalloc: this call needs %zu bytes of scratch, more than "
                "the %zu the library holds per GPU; use moe_fp8_moe_forward_ex with a workspace",
                need, kNoAllocScratchBytes);
    const int rc = scratch_address(as_stream(stream), &workspace);
    if (rc) return rc;
    workspace_bytes = kNoAllocScratchBytes;
  }
  MOE_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "moe_fp8_moe_forward: workspace of %zu bytes needed, %zu given", need,
              workspace_bytes);
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
              "moe_fp8_moe_forward: workspace must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  float* h = static_cast<float*>(workspace);
  const int ids64 = ids_dtype == MOE_I64;
  const int wbf16 = w_dtype == MOE_BF16;
  const int64_t pairs = static_cast<int64_t>(tokens) * top_k;
  if (use_grouped(tokens, hidden, mode)) {
    MOE_REQUIRE(n_experts <= 4096 && pairs <= (1LL << 24) && tokens <= 65535,
                "moe_fp8_moe_forward: grouped path limits: n_experts <= 4096, tokens <= 65535");
    return launch_grouped(static_cast<const uint16_t*>(x), ids, ids64, weights, wbf16, tokens,
                          top_k, static_cast<const uint8_t*>(w13), s13,
                          static_cast<const uint8_t*>(w2), s2, es, n_experts, hidden, inter,
                          static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(out),
                          static_cast<char*>(workspace), s);
  }
  MOE_REQUIRE(pairs <= 65535LL, "moe_fp8_moe_forward: too many (token, expert) pairs (%lld)",
              (long long)pairs);
  if (mode == 3) {
    MOE_REQUIRE(!sh && !rt, "moe_fp8_moe_forward: mode 3 (bf16 activations) carries no shared "
                            "expert or router");
    return launch_gemv_a16(static_cast<const uint16_t*>(x), ids, ids64, weights, wbf16, tokens,
                           top_k, static_cast<const uint8_t*>(w13), s13,
                           static_cast<const uint8_t*>(w2), s2, es, n_experts, hidden, inter,
                           static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(out), h,
                           s);
  }
  // the shared expert rides along (the down workgroup's ceil(top_k/2) + 1
  // waves fit its launch bounds for every top_k)
  *fused = sh != nullptr;
  if (rt) {
    MOE_REQUIRE(tokens <= kGemvMaxTokens && !sh,
                "moe_router_fp8_moe_forward: 1 to %d tokens, no shared expert", kGemvMaxTokens);
    const int rc = launch_router_logits(x, rt->w_gate, rt->bias, tokens, hidden, n_experts,
                                        rt->bf16_logits, rt->logits, s);
    if (rc) return rc;
  }
  return launch_gemv(static_cast<const uint16_t*>(x), ids, ids64, weights, wbf16, tokens, top_k,
                     static_cast<const uint8_t*>(w13), s13, static_cast<const uint8_t*>(w2), s2,
                     es, n_experts, hidden, inter, static_cast<const uint16_t*>(residual),
                     static_cast<uint16_t*>(out), h, sh, s, rt);
}

extern "C" int moe_fp8_moe_forward_ex(const void* x, const void* ids, int32_t ids_dtype,
                                      const void* weights, int32_t w_dtype, int32_t tokens,
                                      int32_t top_k, const void* w13, const float* s13,
                                      const void* w2, const float* s2, int32_t n_experts,
                                      int32_t hidden, int32_t inter,
                                      const moe_expert_strides* strides,
                                      const void* residual, void* out,
                                      void* workspace, size_t workspace_bytes, int32_t mode,
                                      void* stream) {
  bool fused;
  return forward_impl(x, ids, ids_dtype, weights, w_dtype, tokens, top_k, w13, s13, w2, s2,
                      n_experts, hidden, inter, strides, residual, out, workspace, workspace_bytes,
                      mode, nullptr, &fused, stream);
}

extern "C" int moe_router_fp8_moe_forward(const void* x, const void* w_gate, const float* bias,
                                          int32_t logit_dtype, int32_t tokens, int32_t hidden,
                                          int32_t n_experts, int32_t top_k, float* logits,
                                          int32_t* ids, float* weights, const void* w13,
                                          const float* s13, const void* w2, const float* s2,
                                          int32_t inter, const moe_expert_strides* strides,
                                          const void* residual, void* out, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  MOE_REQUIRE(tokens >= 1 && tokens <= kGemvMaxTokens,
              "moe_router_fp8_moe_forward: need 1 <= tokens <= %d", kGemvMaxTokens);
  MOE_REQUIRE(x && w_gate && logits && ids && weights, "moe_router_fp8_moe_forward: NULL pointer");
  MOE_REQUIRE(logit_dtype == MOE_F32 || logit_dtype == MOE_BF16,
              "moe_router_fp8_moe_forward: logit_dtype must be MOE_F32 or MOE_BF16");
  MOE_REQUIRE(top_k >= 1 && top_k <= kMaxK && top_k <= n_experts && n_experts <= 1024,
              "moe_router_fp8_moe_forward: need 1 <= top_k <= min(%d, n_experts), "
              "n_experts <= 1024", kMaxK);
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(w_gate) % 16 == 0,
              "moe_router_fp8_moe_forward: w_gate must be 16-byte aligned");
  const RouterTopK rt{w_gate, bias, logit_dtype == MOE_BF16 ? 1 : 0, logits, ids, weights};
  bool fused;
  // mode 1: the per-pair GEMV kernels, whose gate/up launch makes the top-k;
  // every check of the expert call runs before the logits launch is enqueued
  return forward_impl(x, ids, MOE_I32, weights, MOE_F32, tokens, top_k, w13, s13, w2, s2, n_experts,
                      hidden, inter, strides, residual, out, workspace, workspace_bytes, 1,
                      nullptr, &fused, stream, false, &rt);
}

extern "C" size_t moe_fp8_moe_block_workspace(int32_t tokens, int32_t top_k, int32_t n_experts,
                                              int32_t hidden, int32_t inter,
                                              int32_t shared_inter) {
  const size_t base = align256(moe_fp8_moe_workspace(tokens, top_k, n_experts, hidden, inter));
  if (tokens <= 0 || shared_inter <= 0) return base;
  return base + align256(static_cast<size_t>(tokens) * shared_inter * sizeof(uint16_t)) +
         align256(static_cast<size_t>(tokens) * sizeof(float));
}

extern "C" int moe_fp8_moe_block_forward(const void* x, const void* ids, int32_t ids_dtype,
                                         const void* weights, int32_t w_dtype, int32_t tokens,
                                         int32_t top_k, const void* w13, const float* s13,
                                         const void* w2, const float* s2, int32_t n_experts,
                                         int32_t hidden, int32_t inter,
                                         const moe_expert_strides* strides,
                                         const moe_shared_expert* shared, const void* residual,
                                         void* out, void* workspace, size_t workspace_bytes,
                                         int32_t mode, void* stream) {
  MOE_REQUIRE(tokens >= 0, "moe_fp8_moe_block_forward: tokens < 0");
  MOE_REQUIRE(shared != nullptr, "moe_fp8_moe_block_forward: NULL shared expert");
  const int32_t Is = shared->inter;
  MOE_REQUIRE(Is >= 128 && Is % 128 == 0,
              "moe_fp8_moe_block_forward: shared inter must be a positive multiple of 128");
  if (tokens > 0) {
    MOE_REQUIRE(shared->w_gate && shared->w_up && shared->w_down && shared->w_sgate,
                "moe_fp8_moe_block_forward: NULL shared expert weight");
    MOE_REQUIRE(reinterpret_cast<uintptr_t>(shared->w_gate) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(shared->w_up) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(shared->w_down) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(shared->w_sgate) % 16 == 0,
                "moe_fp8_moe_block_forward: shared expert weights must be 16-byte aligned");
    const size_t need = moe_fp8_moe_block_workspace(tokens, top_k, n_experts, hidden, inter, Is);
    MOE_REQUIRE(workspace != nullptr && workspace_bytes >= need,
                "moe_fp8_moe_block_forward: workspace of %zu bytes needed, %zu given", need,
                workspace_bytes);
  }
  bool fused = false;
  if (tokens == 0)                   // preconditions only; an empty call touches nothing
    return forward_impl(x, ids, ids_dtype, weights, w_dtype, tokens, top_k, w13, s13, w2, s2,
                        n_experts, hidden, inter, strides, residual, out, workspace,
                        workspace_bytes, mode, nullptr, &fused, stream);
  // workspace: the routed call's, then act [T, Is] bf16, then sig [T] f32
  char* ws = static_cast<char*>(workspace);
  const size_t base = align256(moe_fp8_moe_workspace(tokens, top_k, n_experts, hidden, inter));
  uint16_t* act = reinterpret_cast<uint16_t*>(ws + base);
  float* sig = reinterpret_cast<float*>(
      ws + base + align256(static_cast<size_t>(tokens) * Is * sizeof(uint16_t)));
  const SharedRefs sh{static_cast<const uint16_t*>(shared->w_gate),
                      static_cast<const uint16_t*>(shared->w_up),
                      static_cast<const uint16_t*>(shared->w_down),
                      static_cast<const uint16_t*>(shared->w_sgate), Is, act, sig};
  if (mode != 3 && !use_grouped(tokens, hidden, mode) && tokens <= kCarrySharedMaxTokens) {
    // decode: the shared expert rides in the two GEMV launches, residual last
    const int rc = forward_impl(x, ids, ids_dtype, weights, w_dtype, tokens, top_k, w13, s13,
                                w2, s2, n_experts, hidden, inter, strides, residual, out,
                                workspace, base, mode, &sh, &fused, stream);
    MOE_REQUIRE(rc != MOE_OK || fused,
                "moe_fp8_moe_block_forward: the GEMV launches did not carry the shared expert");
    return rc;
  }
  // otherwise: routed experts into out, then the shared expert adds to it in place
  int rc = forward_impl(x, ids, ids_dtype, weights, w_dtype, tokens, top_k, w13, s13, w2, s2,
                        n_experts, hidden, inter, strides, nullptr, out, workspace, base, mode,
                        nullptr, &fused, stream);
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
  rc = launch_shared_gate_up(static_cast<const uint16_t*>(x), sh.wg, sh.wu, sh.wsg, tokens, hidden,
                             Is, act, sig, s);
  if (rc) return rc;
  return launch_shared_down(act, sig, sh.wd, tokens, hidden, Is, static_cast<const uint16_t*>(out),
                            static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(out), s);
}

extern "C" int moe_fp8_moe_forward(const void* x, const void* ids, int32_t ids_dtype,
                                   const void* weights, int32_t w_dtype, int32_t tokens,
                                   int32_t top_k, const void* w13, const float* s13,
                                   const void* w2, const float* s2, int32_t n_experts,
                                   int32_t hidden, int32_t inter, void* out, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  return moe_fp8_moe_forward_ex(x, ids, ids_dtype, weights, w_dtype, tokens, top_k, w13, s13, w2,
                                s2, n_experts, hidden, inter, nullptr, nullptr, out, workspace,
                                workspace_bytes, 0, stream);
}


extern "C" int moe_fp8_moe_forward_noalloc(const void* x, const void* ids, int32_t ids_dtype,
                                           const void* weights, int32_t w_dtype, int32_t tokens,
                                           int32_t top_k, const void* w13, const float* s13,
                                           const void* w2, const float* s2, int32_t n_experts,
                                           int32_t hidden, int32_t inter,
                                           const moe_expert_strides* strides,
                                           const void* residual, void* out, int32_t mode,
                                           void* stream) {
  bool fused;
  return forward_impl(x, ids, ids_dtype, weights, w_dtype, tokens, top_k, w13, s13, w2, s2,
                      n_experts, hidden, inter, strides, residual, out, nullptr, 0, mode, nullptr,
                      &fused, stream, /*static_scratch=*/true);
}

#if defined(MOE_PHASE_MARKS)
// The marks build's reader (no counterpart in the reference, not part of
// the product library): copies the first n words of the phase marks,
// [kernel: gate/up, down][workgroup][wave][mark], to host memory.
extern "C" int moe_phase_marks_read(uint64_t* dst, int32_t n) {
  if (!dst || n < 0 || n > static_cast<int32_t>(sizeof(g_phase_marks) / sizeof(uint64_t)))
    return -1;
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_phase_marks), static_cast<size_t>(n) * 8) ==
                 hipSuccess
             ? 0
             : -1;
}
// The marks' clock in kHz (the device's constant wall clock), or -1.
extern "C" int32_t moe_phase_marks_clock_khz() {
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
    return -1;
  return khz;
}
#endif
