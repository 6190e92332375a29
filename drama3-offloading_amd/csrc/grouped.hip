// Grouped W8A8 expert FFN for many tokens (prefill, batched decode): token
// rows are permuted into per-expert segments (permute.hip), the segments are
// cut into tiles of up to 32 rows, every expert's weights are read from HBM
// once per tile, and the results are un-permuted with the routing weights.
//
//   permute:     the token -> expert grouping and the tile list, and in the
//                same launch x [T, H] bf16 -> xq [T, H] e4m3, xs [T, H/128]
//                (per token; permute.hip).
//   gate/up:     grouped_stream_kernel over (tile, rows of w13) work items,
//                the tile's xq rows gathered by token.  In the GLU form (the
//                default: items of whole 128-column groups) the epilogue
//                forms a = SiLU(gate) * up and quantises it per 128 (aq, as);
//                otherwise it writes h [pos, 2I] float32 in permuted order
//                and a SiLU launch (one wave per permuted row) does the rest.
//   down:        grouped_stream_kernel over (tile, rows of w2) work items on
//                the tile's aq rows: y [pos, H] float32.
//   unpermute:   out[t] = sum_k w[t,k] * y[pos[t,k]] (permute.hip).
//
// The weights are read in either byte order (moe_expert_strides.layout);
// in the MFMA tile order of the packed records each 16-byte load of a wave
// reads 1 KiB contiguous.
//
// MFMA 16x16x128 e4m3 with the same operand roles as the decode GEMV:
// weight rows are the A operand, activations the B operand (one token per B
// column), every lane supplies the same 32-byte reduction slice, block
// scales multiply each 128-deep block result as weight_scale *
// activation_scale, and the blocks are summed in the same order -- so every
// (token, expert) row computed here is bit-identical to the decode GEMV's.
#include <math.h>

#include <type_traits>

#include "common.hpp"
#include "grouped.hpp"

namespace moe {

// ---------------------------------------------------- streamed expert GEMM
//
// One kernel computes both projections.  For the weight rows r of one expert
// and the permuted rows pos of one of its tiles (up to 32 consecutive rows
// of the expert's segment, listed by the permute kernel):
//
//   out[pos][r] = sum over K-blocks kb, in order, of
//                 MFMA(w[e][r][kb], act[pos][kb]) * (w_scale[r/128][kb] * act_scale[pos][kb])
//
//   gate/up:  w = w13 (2I rows, K = H), act = xq gathered by token, out = h
//   down:     w = w2  (H rows,  K = I), act = aq in permuted order,  out = y
//
// A work item is (tile, 64*GPW consecutive weight rows).  One workgroup of 4
// waves takes one item; wave w owns GPW groups of 16 rows.  The wave's
// (K-block, group) units, K-block-major, stream through a ring of RING
// operand registers per lane (16, or 8 for the 8-group shape): unit u+RING
// is loaded as soon as the MFMA of unit u has read its slot, so RING units
// (2 KiB each per wave) stay in flight from the item's first load to its
// last.  The tile's activation rows are
// copied once into LDS by direct global->LDS loads, 16-byte units
// XOR-swizzled by row against bank conflicts, together with their scales and
// the item's weight scales; K beyond 16 blocks is staged 16 blocks at a time.
// Items are dealt to the 8 XCDs in contiguous ranges, so the items of one
// tile mostly share an L2.  Gate/up takes 4 groups per wave (the GLU form),
// down 8 with a ring of 8, each stepping down only for calls too small to
// fill the chip (pick_shape).

constexpr int kTileTok = 32;          // permuted rows per tile (two MFMA column tiles)
constexpr int kColTiles = kTileTok / 16;
constexpr int kWaves = 4;             // waves per workgroup
constexpr int kRing = 16;             // K-block operands in flight per lane
constexpr int kStageBlocks = 16;      // K-blocks of activations staged at a time
constexpr int kStageRowBytes = kStageBlocks * 128;
constexpr int kMaxGPW = 8;            // groups of 16 rows per wave
constexpr int kMaxScaleRows = kMaxGPW / 2;   // 128-row weight-scale rows per item
constexpr int kMinItems = 400;        // fewest work items worth a bigger GPW

// LDS of one workgroup: the activation tile first (the direct loads address
// it from offset 0), then the scales and the tile's token rows.
constexpr int kLdsAct = kTileTok * kStageRowBytes;
constexpr int kLdsActScale = kLdsAct;
constexpr int kLdsWScale = kLdsActScale + 4 * kTileTok * kStageBlocks;
constexpr int kLdsTok = kLdsWScale + 4 * kMaxScaleRows * kStageBlocks;
constexpr int kLdsBytes = kLdsTok + 4 * kTileTok;

struct StreamArgs {
  const uint8_t* act;      // activation rows, e4m3, G*128 bytes each
  const float* act_s;      // their per-128 scales, G per row
  const int32_t* sorted;   // gather only: permuted row -> token * top_k + k
  const int32_t* counts;   // rows per expert
  const int32_t* offsets;  // first permuted row per expert
  const int32_t* tiles;    // (expert, first segment row) per tile
  const int32_t* n_tiles;  // tile count, written by the permute kernel
  const uint8_t* w;        // [E][rows][G*128] e4m3, expert stride w_es bytes
  const float* ws;         // [E][rows/128][G] f32, expert stride s_es floats
  float* out;              // [pairs][rows] f32, permuted order (not in the GLU form)
  int64_t w_es, s_es;
  int32_t top_k, rows, G;
  int32_t tiled;           // w in MFMA tile order (MOE_LAYOUT_TILES), else row-major
  // GLU form (gate/up only): rows = 2 * inter, and instead of `out` the
  // item writes a = SiLU(gate) * up quantised per 128: aq [pairs][inter]
  // e4m3, as [pairs][inter / 128]
  uint8_t* aq;
  float* as;
  int32_t inter;
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 32-byte MFMA operand from two 16-byte units of LDS.
__device__ __forceinline__ v8i lds_op32(const uint8_t* p0, const uint8_t* p1) {
  const u32x4 lo = *reinterpret_cast<const u32x4*>(p0);
  const u32x4 hi = *reinterpret_cast<const u32x4*>(p1);
  return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

// The GLU form of the gate/up projection.  An item takes intermediate
// columns [c, c + 32*GPW) -- whole 128-column groups, GPW >= 4 -- with their
// gate rows (waves 0-1) and their up rows (waves 2-3), so it holds every
// value that SiLU(gate) * up and its per-128 quantisation of those columns
// need.  The row sums go through LDS once (the staging area, free after the
// K loop) and leave as e4m3 codes and scales: no float32 h round trip, no
// separate SiLU launch.  The arithmetic is the decode GEMV's: silu_mul on
// the same row sums, then quantize8_f32, so the codes are identical.
constexpr int kGluPad = 4;            // LDS row padding (floats) of the epilogue tile

template <int RING, int GPW, bool GATHER, bool GLU>
__global__ __launch_bounds__(64 * kWaves) void grouped_stream_kernel(StreamArgs A) {
  static_assert(RING % GPW == 0 && RING <= kRing && GPW <= kMaxGPW, "ring slots per group");
  static_assert(!GLU || GPW >= 4, "the GLU form needs whole 128-column groups per item");
  constexpr int KPP = RING / GPW;                   // K-blocks per pass of the ring
  __shared__ __align__(16) uint8_t smem[kLdsBytes];
  uint8_t* xt = smem;
  float* xst = reinterpret_cast<float*>(smem + kLdsActScale);
  float* wsc = reinterpret_cast<float*>(smem + kLdsWScale);
  int32_t* tok = reinterpret_cast<int32_t*>(smem + kLdsTok);

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4;
  const int col = lane & 15;
  const int G = A.G;
  const int64_t K = static_cast<int64_t>(G) * 128;

  // item of this workgroup: XCD x = blockIdx % 8 takes items [x*n8, (x+1)*n8)
  const int ipt = A.rows / (64 * GPW);
  const int64_t n_items = static_cast<int64_t>(*A.n_tiles) * ipt;
  const int64_t n8 = (n_items + 7) >> 3;
  const int64_t slot8 = blockIdx.x >> 3;
  const int64_t item = static_cast<int64_t>(blockIdx.x & 7) * n8 + slot8;
  if (slot8 >= n8 || item >= n_items) return;      // whole workgroup
  const int64_t tile = item / ipt;
  const int32_t e = A.tiles[2 * tile];
  const int32_t m0 = A.tiles[2 * tile + 1];
  const int32_t seg = A.offsets[e] + m0;            // first permuted row of the tile
  const int32_t ncols = min(kTileTok, A.counts[e] - m0);
  const int nct = (ncols + 15) >> 4;                // column tiles in use
  const int row0 = static_cast<int>(item % ipt) * (64 * GPW);
  // GLU: the item's columns c0..c0+32*GPW-1; waves 0-1 take their gate rows,
  // waves 2-3 their up rows (row inter + c)
  const int c0 = row0 >> 1;
  const int rw = GLU ? (wave >> 1) * A.inter + c0 + (wave & 1) * (16 * GPW)
                     : row0 + wave * (16 * GPW);    // the wave's first row
  // weight-scale rows staged for the item: one contiguous band, or (GLU)
  // the gate band then the up band of nb rows each
  const int nb = GLU ? (32 * GPW + 127) >> 7 : 0;
  const int sb0 = GLU ? c0 >> 7 : row0 >> 7;        // the item's first scale row
  const int nsb = GLU ? 2 * nb : ((row0 + 64 * GPW - 1) >> 7) - sb0 + 1;
  auto scale_row = [&](int slot) {                  // staged slot -> scale row
    return GLU ? (slot < nb ? sb0 + slot : ((A.inter + c0) >> 7) + slot - nb) : sb0 + slot;
  };
  auto scale_slot = [&](int j) {                    // group j of this wave -> staged slot
    return GLU ? (wave >> 1) * nb + (((wave & 1) * (16 * GPW) + 16 * j) >> 7)
               : ((rw + 16 * j) >> 7) - sb0;
  };
  const int Gs = min(G, kStageBlocks);              // K-blocks per staged row
  const int upr = Gs * 8;                           // 16-byte units per staged row
  const int swz = (Gs & 1) ? 7 : 15;                // unit XOR mask (within the row)

  // token rows of the tile (gather form), issued before the weights
  int32_t tokv = 0;
  if (GATHER && threadIdx.x < kTileTok)
    tokv = A.sorted[seg + min(static_cast<int>(threadIdx.x), ncols - 1)] / A.top_k;
  __builtin_amdgcn_sched_barrier(0);

  // fill the ring: unit s = (K-block s / GPW, group s % GPW)
  const OperandWalk ow = operand_walk(rw + col, q, K, A.tiled);
  const uint8_t* wl = A.w + static_cast<int64_t>(e) * A.w_es + ow.off;
  v8i a[RING];
#pragma unroll
  for (int s = 0; s < RING; ++s) {
    const int kb = min(s / GPW, G - 1);
    a[s] = load_op_nt(wl + static_cast<int64_t>(s % GPW) * 16 * K + kb * ow.kstep, ow.half);
  }
  __builtin_amdgcn_sched_barrier(0);

  if (GATHER && threadIdx.x < kTileTok) tok[threadIdx.x] = tokv;
  __syncthreads();

  auto act_row = [&](int r) -> int64_t {
    const int rr = min(r, ncols - 1);
    return GATHER ? static_cast<int64_t>(tok[rr]) : static_cast<int64_t>(seg + rr);
  };
  // K-blocks [16*ph, 16*ph + Gs) of the tile's rows [0, 16*nct) into LDS.
  // Rows past ncols repeat the last row; their columns are never stored.
  auto stage = [&](int ph) {
    const int kb0 = ph * kStageBlocks;
    const int nwin = 2 * nct * Gs;                  // 1 KiB windows, 16 bytes per lane
    for (int win = wave; win < nwin; win += kWaves) {
      const int U = win * 64 + lane;
      const int r = U / upr;
      const int c = (U - r * upr) ^ (r & swz);      // source unit of LDS unit U
      const int kb = kb0 + (c >> 3);
      const uint8_t* src = A.act + act_row(r) * K + (kb < G ? kb * 128 + (c & 7) * 16 : 0);
      __builtin_amdgcn_global_load_lds(src, (lds_ptr_t)(xt + win * 1024), 16, 0, 0);
    }
    for (int i = threadIdx.x; i < 16 * nct * Gs; i += 64 * kWaves) {
      const int kb = kb0 + i % Gs;
      xst[i] = kb < G ? A.act_s[act_row(i / Gs) * G + kb] : 0.0f;
    }
    for (int i = threadIdx.x; i < nsb * Gs; i += 64 * kWaves) {
      const int kb = kb0 + i % Gs;
      wsc[i] = kb < G ? A.ws[static_cast<int64_t>(e) * A.s_es +
                             static_cast<int64_t>(scale_row(i / Gs)) * G + kb]
                      : 0.0f;
    }
    __builtin_amdgcn_s_waitcnt(0);                  // this wave's direct loads landed
    __syncthreads();
  };
  stage(0);

  v4f acc[GPW][kColTiles];
#pragma unroll
  for (int j = 0; j < GPW; ++j)
#pragma unroll
    for (int m = 0; m < kColTiles; ++m) acc[j][m] = v4f{0.f, 0.f, 0.f, 0.f};

  // one pass: K-blocks [p*KPP, p*KPP + KPP) of every group; REFILL issues the
  // loads of the next pass into the slots just read
  auto pass = [&](int p, auto refill) {
    const int kb0 = p * KPP;
    if (kb0 > 0 && (kb0 & (kStageBlocks - 1)) == 0) {   // next 16 K-blocks (K > 2048)
      __syncthreads();
      stage(kb0 / kStageBlocks);
    }
#pragma unroll
    for (int i = 0; i < KPP; ++i) {
      const int kb = kb0 + i;
      if (kb < G) {
        const int kl = kb & (kStageBlocks - 1);
        v8i b[kColTiles];
        float as[kColTiles];
#pragma unroll
        for (int m = 0; m < kColTiles; ++m) {
          if (m < nct) {
            const int R = m * 16 + col;
            const uint8_t* rowp = xt + R * (upr * 16);
            const int c0 = kl * 8 + q * 2;
            const int sw = R & swz;
            b[m] = lds_op32(rowp + ((c0 ^ sw) << 4), rowp + (((c0 + 1) ^ sw) << 4));
            as[m] = xst[R * Gs + kl];
          }
        }
#pragma unroll
        for (int j = 0; j < GPW; ++j) {
          const float wsj = wsc[scale_slot(j) * Gs + kl];
#pragma unroll
          for (int m = 0; m < kColTiles; ++m) {
            if (m < nct) {
              const v4f z = {0.f, 0.f, 0.f, 0.f};
              const v4f d = mfma_e4m3_16x16x128(a[i * GPW + j], b[m], z);
              block_fma(acc[j][m], d, wsj * as[m]);
            }
          }
        }
      }
      if constexpr (decltype(refill)::value) {
        const int kn = min(kb + KPP, G - 1);
#pragma unroll
        for (int j = 0; j < GPW; ++j)
          a[i * GPW + j] = load_op_nt(wl + static_cast<int64_t>(j) * 16 * K + kn * ow.kstep,
                                      ow.half);
      }
    }
  };
  const int npass = (G + KPP - 1) / KPP;
  for (int p = 0; p + 1 < npass; ++p) pass(p, std::true_type{});
  pass(npass - 1, std::false_type{});

  if constexpr (!GLU) {
#pragma unroll
    for (int j = 0; j < GPW; ++j)
#pragma unroll
      for (int m = 0; m < kColTiles; ++m) {
        const int cc = m * 16 + col;
        if (m < nct && cc < ncols)
          *reinterpret_cast<float4*>(A.out + static_cast<int64_t>(seg + cc) * A.rows + rw +
                                     16 * j + 4 * q) =
              make_float4(acc[j][m][0], acc[j][m][1], acc[j][m][2], acc[j][m][3]);
      }
  } else {
    // row sums -> LDS as [gate | up][token][column] (the staging area is
    // free once every wave is past its last K-block)
    constexpr int kCols = 32 * GPW;                 // columns of the item
    constexpr int kStride = kCols + kGluPad;
    static_assert(2 * kTileTok * kStride * 4 <= kLdsBytes, "GLU epilogue tile fits the LDS");
    float* ep = reinterpret_cast<float*>(smem);
    __syncthreads();
    const int half = wave >> 1;
    const int cw = (wave & 1) * (16 * GPW);         // the wave's first column of the item
#pragma unroll
    for (int j = 0; j < GPW; ++j)
#pragma unroll
      for (int m = 0; m < kColTiles; ++m)
        if (m < nct)
          *reinterpret_cast<float4*>(ep + (half * kTileTok + m * 16 + col) * kStride + cw +
                                     16 * j + 4 * q) =
              make_float4(acc[j][m][0], acc[j][m][1], acc[j][m][2], acc[j][m][3]);
    __syncthreads();
    // 16 lanes per (token, 128-column group): 8 columns per lane
    constexpr int kGroups = kCols / 128;
    const int sub = threadIdx.x >> 4;               // 16 rows of 16 lanes
    const int li = threadIdx.x & 15;
    for (int u = sub; u < kTileTok * kGroups; u += 16) {
      const int tt = u / kGroups;
      const int cg = u - tt * kGroups;
      const int cl = cg * 128 + li * 8;             // column within the item
      const float* gp = ep + tt * kStride + cl;
      const float* up = ep + (kTileTok + tt) * kStride + cl;
      const float4 g0 = *reinterpret_cast<const float4*>(gp);
      const float4 g1 = *reinterpret_cast<const float4*>(gp + 4);
      const float4 u0 = *reinterpret_cast<const float4*>(up);
      const float4 u1 = *reinterpret_cast<const float4*>(up + 4);
      const float4 av[2] = {
          make_float4(silu_mul(g0.x, u0.x), silu_mul(g0.y, u0.y), silu_mul(g0.z, u0.z),
                      silu_mul(g0.w, u0.w)),
          make_float4(silu_mul(g1.x, u1.x), silu_mul(g1.y, u1.y), silu_mul(g1.z, u1.z),
                      silu_mul(g1.w, u1.w))};
      const int64_t prow = seg + tt;                // this token's permuted row
      // every lane of the 16 takes part in the group maximum; rows past the
      // tile's tokens store nothing
      quantize8_f32(av, tt < ncols, c0 + cl, A.aq + prow * A.inter,
                    A.as + prow * (A.inter >> 7));
    }
  }
}

// Work-item shapes, in increasing rows per item: (ring slots, groups of 16
// rows per wave).  The last trades ring depth for rows so that the
// accumulators of 8 groups fit beside the ring at 2 waves per SIMD.
struct StreamShape {
  int ring, gpw;
};
constexpr StreamShape kShapes[] = {{16, 1}, {16, 2}, {16, 4}, {8, 8}};
constexpr int kNumShapes = sizeof(kShapes) / sizeof(kShapes[0]);
constexpr int kGateUpShape = 2;       // (16, 4): whole 128-column groups, the GLU form
constexpr int kDownShape = 3;         // (8, 8)
static_assert(kGateUpShape < kNumShapes && kDownShape < kNumShapes, "shape index");

// Expected tile count of P uniform picks over n_experts: each expert's
// pair count n is Poisson(P / n_experts) and takes ceil(n / 32) tiles,
// E[ceil(n / 32)] = sum over j >= 0 of P(n > 32 j).
static double expected_tiles(int64_t P, int32_t n_experts) {
  if (P <= 0) return 0.0;
  const double lam = static_cast<double>(P) / n_experts;
  if (lam > 1000.0) return n_experts * (lam / kTileTok + 0.5);
  double tiles = 0.0, cdf = 0.0, logp = -lam;   // log P(n = 0)
  int n = 0;
  for (int j = 0;; ++j) {
    const int m = kTileTok * j;
    for (; n <= m; ++n) {
      cdf += exp(logp);
      logp += log(lam) - log(static_cast<double>(n + 1));
    }
    const double tail = 1.0 - cdf;
    if (m > lam && tail < 1e-9) break;
    tiles += tail;
  }
  return n_experts * tiles;
}

// Shape for a projection of `rows` weight rows: the biggest up to `target`
// that tiles the rows and still gives kMinItems work items at the expected
// tile count (fewer items than that leave CUs idle: small calls over few
// experts take smaller items).  Bigger items amortise each workgroup's start
// (tile look-up, staging, first loads) and drain; the GLU form needs
// GPW >= 4.  Measured on MI355X over 256 resident experts, top-8, H 2048,
// I 512, T = 17 .. 1024 tokens and every pair of shapes: gate/up (16, 4)
// with down (8, 8) was the fastest pair or within 1.5 % of it at every T.
static int pick_shape(int64_t P, int32_t n_experts, int32_t rows, int target) {
  const double tiles = expected_tiles(P, n_experts);
  int fallback = -1;
  for (int i = target; i >= 0; --i) {
    const int g = kShapes[i].gpw;
    if (rows % (64 * g) != 0) continue;
    fallback = i;
    if (tiles * rows / (64.0 * g) >= kMinItems) return i;
  }
  return fallback < 0 ? 0 : fallback;
}

// Whether the GLU form serves a gate/up projection of this shape: items of
// whole 128-column groups (GPW >= 4) that tile the intermediate columns.
static bool glu_shape(int shape, int32_t inter) {
  const int g = kShapes[shape].gpw;
  return g >= 4 && inter % (32 * g) == 0;
}

template <bool GATHER, bool GLU = false>
static void launch_stream(const StreamArgs& A, int shape, int64_t max_tiles, hipStream_t s) {
  const int64_t items = max_tiles * (A.rows / (64 * kShapes[shape].gpw));
  const dim3 grid(static_cast<unsigned>((items + 7) & ~int64_t{7}));
  const dim3 block(64 * kWaves);
  if constexpr (GLU) {
    if (shape == 2)
      hipLaunchKernelGGL((grouped_stream_kernel<16, 4, GATHER, true>), grid, block, 0, s, A);
    else
      hipLaunchKernelGGL((grouped_stream_kernel<8, 8, GATHER, true>), grid, block, 0, s, A);
    return;
  }
  switch (shape) {
    case 0: hipLaunchKernelGGL((grouped_stream_kernel<16, 1, GATHER, false>), grid, block, 0, s, A); break;
    case 1: hipLaunchKernelGGL((grouped_stream_kernel<16, 2, GATHER, false>), grid, block, 0, s, A); break;
    case 2: hipLaunchKernelGGL((grouped_stream_kernel<16, 4, GATHER, false>), grid, block, 0, s, A); break;
    default: hipLaunchKernelGGL((grouped_stream_kernel<8, 8, GATHER, false>), grid, block, 0, s, A); break;
  }
}

// ------------------------------------------------------ SiLU * up -> e4m3

// One wave per permuted row: a = SiLU(gate) * up quantised per 128, with the
// decode GEMV's arithmetic (its gate/up kernel's silu_mul, its down kernel's
// quantize8_f32) on the same row sums, so both paths give the same codes.
__global__ __launch_bounds__(512) void grouped_silu_kernel(const float* __restrict__ h,
                                                           const int32_t* __restrict__ offsets,
                                                           int32_t n_experts, int32_t inter,
                                                           uint8_t* __restrict__ aq,
                                                           float* __restrict__ as_) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 6);
  if (row >= offsets[n_experts]) return;    // rows of valid pairs only
  const int lane = threadIdx.x & 63;
  const float* hp = h + row * (2 * inter);
  for (int base = 0; base < inter; base += 512) {
    const int j = base + lane * 8;
    const int jj = j < inter ? j : 0;
    float4 hr[4];
    hr[0] = *reinterpret_cast<const float4*>(hp + jj);
    hr[1] = *reinterpret_cast<const float4*>(hp + jj + 4);
    hr[2] = *reinterpret_cast<const float4*>(hp + inter + jj);
    hr[3] = *reinterpret_cast<const float4*>(hp + inter + jj + 4);
    silu_quantize8(hr, j < inter, j, aq + row * inter, as_ + row * (inter >> 7));
  }
}


// --------------------------------------------------------------- driver

GroupedLayout grouped_layout(int32_t tokens, int32_t top_k, int32_t n_experts, int32_t hidden,
                             int32_t inter) {
  GroupedLayout L;
  const int64_t P = static_cast<int64_t>(tokens) * top_k;
  auto align = [](size_t v) { return (v + 255) & ~static_cast<size_t>(255); };
  size_t o = 0;
  const int64_t max_tiles = (P + kTileTok - 1) / kTileTok + n_experts;
  L.counts = o;       o = align(o + sizeof(int32_t) * n_experts);
  L.offsets = o;      o = align(o + sizeof(int32_t) * (n_experts + 1));
  L.sorted = o;       o = align(o + sizeof(int32_t) * P);
  L.pos = o;          o = align(o + sizeof(int32_t) * P);
  L.tiles = o;        o = align(o + sizeof(int32_t) * 2 * max_tiles);
  L.n_tiles = o;      o = align(o + sizeof(int32_t));
  L.xq = o;           o = align(o + static_cast<size_t>(tokens) * hidden);
  L.xs = o;           o = align(o + sizeof(float) * tokens * (hidden / 128));
  L.h = o;            o = align(o + sizeof(float) * P * 2 * inter);
  L.aq = o;           o = align(o + static_cast<size_t>(P) * inter);
  L.as = o;           o = align(o + sizeof(float) * P * (inter / 128));
  L.y = o;            o = align(o + sizeof(float) * P * hidden);
  L.total = o;
  return L;
}

int launch_grouped(const uint16_t* x, const void* ids, int ids64, const void* weights, int wbf16,
                   int32_t tokens, int32_t top_k, const uint8_t* w13, const float* s13,
                   const uint8_t* w2, const float* s2, const moe_expert_strides& es,
                   int32_t n_experts, int32_t hidden, int32_t inter, const uint16_t* residual,
                   uint16_t* out, char* ws, hipStream_t s) {
  const GroupedLayout L = grouped_layout(tokens, top_k, n_experts, hidden, inter);
  int32_t* counts = reinterpret_cast<int32_t*>(ws + L.counts);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + L.offsets);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + L.sorted);
  int32_t* pos = reinterpret_cast<int32_t*>(ws + L.pos);
  uint8_t* xq = reinterpret_cast<uint8_t*>(ws + L.xq);
  float* xs = reinterpret_cast<float*>(ws + L.xs);
  uint8_t* aq = reinterpret_cast<uint8_t*>(ws + L.aq);
  float* as_ = reinterpret_cast<float*>(ws + L.as);
  float* y = reinterpret_cast<float*>(ws + L.y);
  float* h = reinterpret_cast<float*>(ws + L.h);
  int32_t* tiles = reinterpret_cast<int32_t*>(ws + L.tiles);
  int32_t* n_tiles = reinterpret_cast<int32_t*>(ws + L.n_tiles);
  const int64_t P = static_cast<int64_t>(tokens) * top_k;
  const int64_t max_tiles = (P + kTileTok - 1) / kTileTok + n_experts;
  // the permutation and the activation rows' quantisation in one launch
  const QuantRowsJob quant{x, hidden, xq, xs, tokens};
  int rc = launch_permute(ids, ids64, P, n_experts, counts, offsets, sorted, pos, s, tiles, n_tiles,
                          kTileTok, &quant);
  if (rc) return rc;
  StreamArgs gu{};
  gu.act = xq;  gu.act_s = xs;  gu.sorted = sorted;
  gu.counts = counts;  gu.offsets = offsets;  gu.tiles = tiles;  gu.n_tiles = n_tiles;
  gu.w = w13;  gu.ws = s13;  gu.out = h;  gu.w_es = es.w13;  gu.s_es = es.s13;
  gu.top_k = top_k;  gu.rows = 2 * inter;  gu.G = hidden / 128;
  gu.tiled = es.layout == MOE_LAYOUT_TILES;
  gu.aq = aq;  gu.as = as_;  gu.inter = inter;
  const int gu_shape = pick_shape(P, n_experts, gu.rows, kGateUpShape);
  if (glu_shape(gu_shape, inter)) {
    // gate/up, SiLU * up and its quantisation in one launch
    launch_stream<true, true>(gu, gu_shape, max_tiles, s);
    rc = check_launch("moe_fp8_moe_forward(grouped gate/up + SiLU)");
    if (rc) return rc;
  } else {
    launch_stream<true>(gu, gu_shape, max_tiles, s);
    rc = check_launch("moe_fp8_moe_forward(grouped gate/up)");
    if (rc) return rc;
    hipLaunchKernelGGL(grouped_silu_kernel, dim3(static_cast<unsigned>((P + 7) / 8)), dim3(512), 0,
                       s, h, offsets, n_experts, inter, aq, as_);
    rc = check_launch("moe_fp8_moe_forward(grouped silu)");
    if (rc) return rc;
  }
  StreamArgs dn{};
  dn.act = aq;  dn.act_s = as_;  dn.sorted = nullptr;
  dn.counts = counts;  dn.offsets = offsets;  dn.tiles = tiles;  dn.n_tiles = n_tiles;
  dn.w = w2;  dn.ws = s2;  dn.out = y;  dn.w_es = es.w2;  dn.s_es = es.s2;
  dn.top_k = top_k;  dn.rows = hidden;  dn.G = inter / 128;
  dn.tiled = es.layout == MOE_LAYOUT_TILES;
  launch_stream<false>(dn, pick_shape(P, n_experts, dn.rows, kDownShape), max_tiles, s);
  rc = check_launch("moe_fp8_moe_forward(grouped down)");
  if (rc) return rc;
  return launch_unpermute(y, pos, weights, wbf16, tokens, top_k, hidden, residual, out, s);
}

}  // namespace moe
