// Grouped W8A8 expert FFN for many tokens (prefill, batched decode): token
// rows are permuted into per-expert segments (permute.hip), the segments are
// cut into tiles of up to 32 rows, every expert's weights are read from HBM
// once per tile, and the results are un-permuted with the routing weights.
//
//   quant_rows:  x [T, H] bf16 -> xq [T, H] e4m3, xs [T, H/128]   (per token)
//   gateup:      work items (tile, 64 rows of w13), 4 waves x 16 rows each
//                with every K-block of the wave's rows in flight at once; the
//                tile's xq rows are staged in LDS for the 4 waves.  A fixed
//                grid of workgroups strides over the items, whose count the
//                permute kernel leaves on the device.  h [pos, 2I] float32 in
//                permuted order.
//   silu:        one wave per permuted row: a = SiLU(gate) * up, quantised
//                per 128 (aq, as) -- the decode GEMV's own function.
//   down:        work items (tile, 64 rows of w2) the same way, the tile's aq
//                rows staged in LDS.  y [pos, H] float32.
//   unpermute:   out[t] = sum_k w[t,k] * y[pos[t,k]] (permute.hip).
//
// MFMA 16x16x128 e4m3 with the same operand roles as the decode GEMV:
// weight rows are the A operand, activations the B operand (one token per B
// column), every lane supplies the same 32-byte reduction slice, block
// scales multiply each 128-deep block result as weight_scale *
// activation_scale, and the blocks are summed in the same order -- so every
// (token, expert) row computed here is bit-identical to the decode GEMV's.
#include "common.hpp"
#include "grouped.hpp"

namespace moe {


// --------------------------------------------------------------- quant x

__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t* __restrict__ x,
                                                         int32_t hidden, uint8_t* __restrict__ xq,
                                                         float* __restrict__ xs) {
  // one workgroup per token; 16 threads x 8 values per 128-group
  const int64_t t = blockIdx.x;
  const uint16_t* xr = x + t * hidden;
  for (int base = 0; base < hidden; base += 2048) {
    const int i = base + threadIdx.x * 8;
    float v[8];
    float amax = 0.0f;
    if (i < hidden) {
      const uint4 raw = *reinterpret_cast<const uint4*>(xr + i);
      const uint32_t r[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = __uint_as_float(r[j] << 16);
        v[2 * j + 1] = __uint_as_float(r[j] & 0xffff0000u);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    if (i < hidden) {
      const float s = act_scale(amax);
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) lo |= quant_e4m3(v[j], s) << (8 * j);
#pragma unroll
      for (int j = 0; j < 4; ++j) hi |= quant_e4m3(v[4 + j], s) << (8 * j);
      *reinterpret_cast<uint2*>(xq + t * hidden + i) = make_uint2(lo, hi);
      if ((threadIdx.x & 15) == 0) xs[t * (hidden >> 7) + (i >> 7)] = s;
    }
  }
}

// ------------------------------------------------------- work items
//
// A tile is up to kTileTok consecutive rows (tokens) of one expert's segment
// (listed by the permute kernel).  A work item is (tile, group of 64 weight
// rows): 4 waves x 16 rows, every K-block of a wave's rows loaded at once
// (all of the item's weight bytes in flight), the tile's activations staged
// once in LDS for the 4 waves.  Two such workgroups fit on a CU, so one
// streams weights while the other stages and computes.  Grids are a fixed number of workgroups that
// stride over the items, whose count is read on the device.

constexpr int kTileTok = 32;         // tokens per tile (two MFMA column tiles)
constexpr int kColTiles = kTileTok / 16;
constexpr int kItemWaves = 4;        // 64 weight rows per work item
constexpr int kKChunk = 16;          // K-blocks of 128 in flight per lane (2048 columns)
constexpr int kKHalf = kKChunk / 2;  // K-blocks of activations staged at a time
constexpr int kItemWGs = 1024;       // workgroups striding over the items (2 resident per CU)
constexpr int kStagePad = 16;        // LDS row padding (bytes) against bank conflicts
constexpr int kDownKChunk = 4;       // K-blocks per chunk in the down kernel (inter 512 = 1 chunk)

// (expert, first segment row, segment offset, rows in the tile) of a tile.
struct TileInfo {
  int32_t e = 0, m0 = 0, off = 0, ncols = 0;
  __device__ __forceinline__ void load(const int32_t* tiles, const int32_t* offsets,
                                       const int32_t* counts, int64_t tile) {
    e = tiles[2 * tile];
    m0 = tiles[2 * tile + 1];
    off = offsets[e];
    ncols = min(kTileTok, counts[e] - m0);
  }
};

// Staging of an activation tile, rows [0, kTileTok) x 16-byte units
// [0, UNITS), in two steps so that the loads can be issued early:
// stage_load reads row r from src_row(r), stage_store writes it to LDS (or
// zeros when row_live(r) is false).
template <int UNITS>
struct Stage {
  static constexpr int kPer = kTileTok * UNITS / (64 * kItemWaves);
  u32x4 v[kPer];

  template <typename SrcRow>
  __device__ __forceinline__ void load(SrcRow src_row) {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = threadIdx.x + u * 64 * kItemWaves;
      v[u] = *reinterpret_cast<const u32x4*>(src_row(i / UNITS) + (i % UNITS) * 16);
    }
  }
  template <int PITCH, typename Live>
  __device__ __forceinline__ void store(uint8_t (*dst)[PITCH], Live row_live) const {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = threadIdx.x + u * 64 * kItemWaves;
      *reinterpret_cast<u32x4*>(&dst[i / UNITS][(i % UNITS) * 16]) =
          row_live(i / UNITS) ? v[u] : u32x4{0u, 0u, 0u, 0u};
    }
  }
};

// --------------------------------------------------------------- gate/up

// h[pos][r] for the 2I weight rows r and the tile's rows pos: exactly the
// decode GEMV's per-row arithmetic (block results scaled weight-scale first,
// summed with one fma per block in K order).
__global__ __launch_bounds__(64 * kItemWaves) void grouped_gateup_kernel(
    const uint8_t* __restrict__ xq, const float* __restrict__ xs,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_pairs, const int32_t* __restrict__ tiles,
    const int32_t* __restrict__ n_tiles, int32_t top_k, const uint8_t* __restrict__ w13,
    const float* __restrict__ s13, int64_t w13_es, int64_t s13_es, int32_t hidden, int32_t inter,
    float* __restrict__ h) {
  __shared__ __align__(16) uint8_t xt[kTileTok][kKHalf * 128 + kStagePad];
  __shared__ float xst[kTileTok][kKHalf];
  __shared__ int32_t tok[kTileTok];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4;
  const int col = lane & 15;
  const int G = hidden >> 7;
  const int rows2 = 2 * inter;
  const int groups = rows2 / (16 * kItemWaves);
  const int64_t n_items = static_cast<int64_t>(*n_tiles) * groups;
  // the tile entry of the next item is fetched while this one runs
  TileInfo nxt;
  if (blockIdx.x < n_items) nxt.load(tiles, offsets, counts, blockIdx.x / groups);
  for (int64_t item = blockIdx.x; item < n_items; item += gridDim.x) {
    const TileInfo cur = nxt;
    if (item + gridDim.x < n_items) nxt.load(tiles, offsets, counts, (item + gridDim.x) / groups);
    const int r0 = static_cast<int>(item % groups) * (16 * kItemWaves) + wave * 16;
    const int32_t e = cur.e;
    const int32_t m0 = cur.m0;
    const int32_t off = cur.off;
    const int32_t ncols = cur.ncols;
    const int nct = (ncols + 15) >> 4;                 // column tiles in use
    const uint8_t* wrow = w13 + static_cast<int64_t>(e) * w13_es +
                          static_cast<int64_t>(r0 + col) * hidden + q * 32;
    const float* srow = s13 + static_cast<int64_t>(e) * s13_es + static_cast<int64_t>(r0 >> 7) * G;
    __syncthreads();                 // the previous item is done with tok / xt
    if (threadIdx.x < kTileTok)
      tok[threadIdx.x] =
          threadIdx.x < ncols ? sorted_pairs[off + m0 + threadIdx.x] / top_k : -1;
    v4f acc[kColTiles];
#pragma unroll
    for (int m = 0; m < kColTiles; ++m) acc[m] = v4f{0.f, 0.f, 0.f, 0.f};
    __syncthreads();                 // tok visible
    for (int k0 = 0; k0 < G; k0 += kKChunk) {
      // activations of the first half go out before the weights: loads
      // retire in issue order, so they can be staged while the weights travel
      Stage<kKHalf * 128 / 16> st;
      auto src_row = [&](int kh) {
        return [&, kh](int r) {
          const int32_t tc = tok[r];
          const int kb = kh * 128;
          return xq + static_cast<int64_t>(tc >= 0 ? tc : 0) * hidden + (kb < hidden ? kb : 0);
        };
      };
      st.load(src_row(k0));
      v8i a[kKChunk];
#pragma unroll
      for (int c = 0; c < kKChunk; ++c) {
        const int g = k0 + c < G ? k0 + c : G - 1;
        a[c] = load_op32_nt(wrow + g * 128);
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int kh = k0 + half * kKHalf;            // first K-block of this half
        if (half > 0) {
          __syncthreads();           // the first half's xt reads are done
          st.load(src_row(kh));
        } else if (k0 > 0) {
          __syncthreads();           // the previous chunk's xt reads are done
        }
        st.store(xt, [&](int r) { return tok[r] >= 0 && kh < G; });
        for (int i = threadIdx.x; i < kTileTok * kKHalf; i += 64 * kItemWaves) {
          const int cc = i / kKHalf, g = i % kKHalf;
          const int32_t t2 = tok[cc];
          xst[cc][g] = (t2 >= 0 && kh + g < G) ? xs[static_cast<int64_t>(t2) * G + kh + g] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < kKHalf; ++c) {
          if (kh + c < G) {
#pragma unroll
            for (int m = 0; m < kColTiles; ++m) {
              if (m < nct) {
                const v8i b = load_op32(&xt[m * 16 + col][c * 128 + q * 32]);
                const v4f z = {0.f, 0.f, 0.f, 0.f};
                const v4f d = mfma_e4m3_16x16x128(a[half * kKHalf + c], b, z);
                const float sc = srow[kh + c] * xst[m * 16 + col][c];
                block_fma(acc[m], d, sc);
              }
            }
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < kColTiles; ++m) {
      const int cc = m * 16 + col;
      if (cc < ncols)
        *reinterpret_cast<float4*>(h + static_cast<int64_t>(off + m0 + cc) * rows2 + r0 + 4 * q) =
            make_float4(acc[m][0], acc[m][1], acc[m][2], acc[m][3]);
    }
  }
}

// ------------------------------------------------------ SiLU * up -> e4m3

// One wave per permuted row: a = SiLU(gate) * up quantised per 128, the
// decode GEMV's silu_quantize8 on the same h values.
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

// --------------------------------------------------------------- down

// y[pos][c] for the H output rows c: w2 rows are the A operand, the tile's
// aq rows (staged in LDS) the B operand.
__global__ __launch_bounds__(64 * kItemWaves) void grouped_down_kernel(
    const uint8_t* __restrict__ aq, const float* __restrict__ as_,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ n_tiles,
    const uint8_t* __restrict__ w2, const float* __restrict__ s2, int64_t w2_es, int64_t s2_es,
    int32_t hidden, int32_t inter, float* __restrict__ y) {
  __shared__ __align__(16) uint8_t at[kTileTok][kDownKChunk * 128 + kStagePad];
  __shared__ float ast[kTileTok][kDownKChunk];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4;
  const int col = lane & 15;
  const int Gi = inter >> 7;
  const int groups = hidden / (16 * kItemWaves);
  const int64_t n_items = static_cast<int64_t>(*n_tiles) * groups;
  TileInfo nxt;
  if (blockIdx.x < n_items) nxt.load(tiles, offsets, counts, blockIdx.x / groups);
  for (int64_t item = blockIdx.x; item < n_items; item += gridDim.x) {
    const TileInfo cur = nxt;
    if (item + gridDim.x < n_items) nxt.load(tiles, offsets, counts, (item + gridDim.x) / groups);
    const int c0 = static_cast<int>(item % groups) * (16 * kItemWaves) + wave * 16;
    const int32_t e = cur.e;
    const int32_t m0 = cur.m0;
    const int32_t off = cur.off;
    const int32_t ncols = cur.ncols;
    const int nct = (ncols + 15) >> 4;
    const uint8_t* wrow = w2 + static_cast<int64_t>(e) * w2_es +
                          static_cast<int64_t>(c0 + col) * inter + q * 32;
    const float* srow = s2 + static_cast<int64_t>(e) * s2_es + static_cast<int64_t>(c0 >> 7) * Gi;
    v4f acc[kColTiles];
#pragma unroll
    for (int m = 0; m < kColTiles; ++m) acc[m] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < Gi; k0 += kDownKChunk) {
      v8i a[kDownKChunk];
#pragma unroll
      for (int c = 0; c < kDownKChunk; ++c) {
        const int g = k0 + c < Gi ? k0 + c : Gi - 1;
        a[c] = load_op32_nt(wrow + g * 128);
      }
      __syncthreads();               // the previous item / chunk is done with at
      {
        Stage<kDownKChunk * 128 / 16> st;
        st.load([&](int r) {
          const int kb = k0 * 128;
          return aq + static_cast<int64_t>(off + m0 + (r < ncols ? r : 0)) * inter +
                 (kb < inter ? kb : 0);
        });
        st.store(at, [&](int r) { return r < ncols; });
      }
      for (int i = threadIdx.x; i < kTileTok * kDownKChunk; i += 64 * kItemWaves) {
        const int cc = i / kDownKChunk, g = i % kDownKChunk;
        ast[cc][g] = (cc < ncols && k0 + g < Gi)
                         ? as_[static_cast<int64_t>(off + m0 + cc) * Gi + k0 + g] : 0.0f;
      }
      __syncthreads();
#pragma unroll
      for (int c = 0; c < kDownKChunk; ++c) {
        if (k0 + c < Gi) {
#pragma unroll
          for (int m = 0; m < kColTiles; ++m) {
            if (m < nct) {
              const v8i b = load_op32(&at[m * 16 + col][c * 128 + q * 32]);
              const v4f z = {0.f, 0.f, 0.f, 0.f};
              const v4f d = mfma_e4m3_16x16x128(a[c], b, z);
              const float sc = srow[k0 + c] * ast[m * 16 + col][c];
              block_fma(acc[m], d, sc);
            }
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < kColTiles; ++m) {
      const int cc = m * 16 + col;
      if (cc < ncols)
        *reinterpret_cast<float4*>(y + static_cast<int64_t>(off + m0 + cc) * hidden + c0 + 4 * q) =
            make_float4(acc[m][0], acc[m][1], acc[m][2], acc[m][3]);
    }
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
  int rc = launch_permute(ids, ids64, P, n_experts, counts, offsets, sorted, pos, s, tiles, n_tiles,
                          kTileTok);
  if (rc) return rc;
  hipLaunchKernelGGL(quant_rows_kernel, dim3(tokens), dim3(256), 0, s, x, hidden, xq, xs);
  rc = check_launch("moe_fp8_moe_forward(quant)");
  if (rc) return rc;
  const int64_t gu_items = max_tiles * ((2 * inter) / (16 * kItemWaves));
  hipLaunchKernelGGL(grouped_gateup_kernel,
                     dim3(static_cast<unsigned>(gu_items < kItemWGs ? gu_items : kItemWGs)),
                     dim3(64 * kItemWaves), 0, s, xq, xs, counts, offsets, sorted, tiles, n_tiles,
                     top_k, w13, s13, es.w13, es.s13, hidden, inter, h);
  rc = check_launch("moe_fp8_moe_forward(grouped gate/up)");
  if (rc) return rc;
  hipLaunchKernelGGL(grouped_silu_kernel, dim3(static_cast<unsigned>((P + 7) / 8)), dim3(512), 0, s,
                     h, offsets, n_experts, inter, aq, as_);
  rc = check_launch("moe_fp8_moe_forward(grouped silu)");
  if (rc) return rc;
  const int64_t dn_items = max_tiles * (hidden / (16 * kItemWaves));
  hipLaunchKernelGGL(grouped_down_kernel,
                     dim3(static_cast<unsigned>(dn_items < kItemWGs ? dn_items : kItemWGs)),
                     dim3(64 * kItemWaves), 0, s, aq, as_, counts, offsets, tiles, n_tiles, w2, s2,
                     es.w2, es.s2, hidden, inter, y);
  rc = check_launch("moe_fp8_moe_forward(grouped down)");
  if (rc) return rc;
  return launch_unpermute(y, pos, weights, wbf16, tokens, top_k, hidden, residual, out, s);
}

}  // namespace moe
