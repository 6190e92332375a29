// A bf16 matrix-vector product for up to 4 tokens (and, on the matrix
// cores, a skinny product for 5 to 128): y[t] = x[t] W^T with W
// [out, in] in nn.Linear layout, every output the f32 sum of its row's
// products rounded once to bf16.  The decode benchmark's stand-in for the
// non-expert compute between two MoE layers (one [2048, 2048] matrix per
// layer) runs on it: at one token the product is one pass over 8 MiB of
// weights, HBM-bound, and the MoE layer after it cannot start before its
// last output is written.
//
// Each wave takes NR consecutive rows; lane l sums the row's 16-byte slices
// l, l + 64, l + 128, ... in order with one fma per product, and the 64
// lane sums are added by DPP (the order of rows_dot_bf16, the shared
// expert's dot product).  All of a lane's slices of its rows are loaded
// before any is used, so every wave issues its whole share of the matrix
// at once: x first (every wave reads it, from L2), then the weights with
// nontemporal loads (read once).
//
// With an addend r (moe_linear_bf16's x_add), the product is of bf16(x + r),
// each element's float sum rounded once to bf16 (a torch add of two bf16
// tensors): a decode step whose residual add sits between two layers'
// products folds it into the second one's loads.  r is loaded beside x and
// the sums are formed after the weight loads are issued; forming them
// before (x's round trip ahead of the weights') cost the saved launch back.
#include "shared.hpp"

namespace moe {

// bf16(a + b) of the 8 bf16 pairs of two 16-byte slices, each sum in float
// rounded once to nearest even.
__device__ __forceinline__ u32x4 add8_bf16(u32x4 a, u32x4 b) {
  const uint32_t av[4] = {a.x, a.y, a.z, a.w};
  const uint32_t bv[4] = {b.x, b.y, b.z, b.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = f32_to_bf16(__uint_as_float(av[i] << 16) + __uint_as_float(bv[i] << 16));
    const uint32_t hi = f32_to_bf16(__uint_as_float(av[i] & 0xffff0000u) +
                                    __uint_as_float(bv[i] & 0xffff0000u));
    o[i] = lo | (hi << 16);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

// One wave per workgroup, one row per wave by default: a graph of
// 1-token calls over 40 layers' [2048, 2048] matrices (MI355X) took 3.55 us
// per call with 1, 2 or 4 one-row waves per workgroup (3.55 / 3.59 / 3.60),
// 3.89 with two rows per wave and 4.54 with four, against 6.9 us for
// torch.mv; loading the weights with ordinary loads and x after them took
// 3.85.
constexpr int kLinearWaves = 1;      // waves per workgroup
constexpr int kLinearMaxTokens = 4;

template <int NR, int TB, bool ADD>
__global__ __launch_bounds__(64 * kLinearWaves) void linear_bf16_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ xa,
    const uint16_t* __restrict__ w, int32_t tokens, int32_t in, int32_t out,
    uint16_t* __restrict__ y) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r0 = (static_cast<int>(blockIdx.x) * kLinearWaves + wave) * NR;
  if (r0 >= out) return;                       // the whole wave; no barrier below
  const uint16_t* rows[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) rows[i] = w + static_cast<int64_t>(min(r0 + i, out - 1)) * in;
  constexpr int U = 4;                         // slices per lane per row in flight
  const int n16 = in >> 3;
  float acc[NR][TB];
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int t = 0; t < TB; ++t) acc[i][t] = 0.0f;
  for (int c0 = 0; c0 < n16; c0 += 64 * U) {
    u32x4 xv[TB][U], av[ADD ? TB : 1][U], wv[U][NR];
#pragma unroll
    for (int t = 0; t < TB; ++t)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = min(c0 + u * 64 + lane, n16 - 1);
        const int64_t o = static_cast<int64_t>(min(t, tokens - 1)) * in + c * 8;
        xv[t][u] = load16(x + o);
        if constexpr (ADD) av[t][u] = load16(xa + o);
      }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(c0 + u * 64 + lane, n16 - 1);
#pragma unroll
      for (int i = 0; i < NR; ++i)
        wv[u][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rows[i] + c * 8));
    }
    if constexpr (ADD) {                         // after every load is issued
#pragma unroll
      for (int t = 0; t < TB; ++t)
#pragma unroll
        for (int u = 0; u < U; ++u) xv[t][u] = add8_bf16(xv[t][u], av[t][u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (c0 + u * 64 + lane >= n16) continue;
#pragma unroll
      for (int t = 0; t < TB; ++t)
#pragma unroll
        for (int i = 0; i < NR; ++i) acc[i][t] = dot8_bf16(wv[u][i], xv[t][u], acc[i][t]);
    }
  }
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int t = 0; t < TB; ++t) acc[i][t] = wave_sum_f32(acc[i][t]);
  if (lane == 0) {
#pragma unroll
    for (int t = 0; t < TB; ++t)
#pragma unroll
      for (int i = 0; i < NR; ++i)
        if (t < tokens && r0 + i < out)
          y[static_cast<int64_t>(t) * out + r0 + i] = f32_to_bf16(acc[i][t]);
  }
}

// 5 to 128 tokens: the product on the bf16 matrix cores.  A workgroup takes
// 16 rows of W and TT tiles of 16 tokens; its kLinMmaWaves waves split K,
// wave v taking the 64-wide chunks v, v + kLinMmaWaves, ...  Lane (q, i) =
// (lane / 16, lane % 16) loads 32 bytes of row i, K 16q .. 16q + 15 of a
// chunk (a row's 128 bytes are read whole by its four lanes), and the same
// K of token i's row of x; the chunk is two MFMAs, one on each 16-byte half,
// so every product of the chunk is formed once.  The waves' partial tiles
// are added in wave order through LDS and rounded once to bf16.  The sum's
// order differs from the one-token kernel's (the matrix cores add inside
// each MFMA), so the outputs agree with the float64 product to within one
// bf16 step, as that kernel's do.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ v4f mfma_bf16_16x16x32(u32x4 a, u32x4 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

constexpr int kLinMmaWaves = 8;         // K slices per workgroup
constexpr int kLinMmaChunks = 4;        // 64-wide K chunks per wave in flight
constexpr int kLinMmaMaxTokens = 128;

template <int TT>
__global__ __launch_bounds__(64 * kLinMmaWaves) void linear_bf16_mma_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int32_t tokens, int32_t in,
    int32_t out, uint16_t* __restrict__ y) {
  __shared__ float part[kLinMmaWaves][TT][16][17];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = lane & 15, q = lane >> 4;
  const int r0 = static_cast<int>(blockIdx.x) * 16;
  const int t0 = static_cast<int>(blockIdx.y) * 16 * TT;
  const int nchunk = in >> 6;
  const uint16_t* wrow = w + static_cast<int64_t>(r0 + i) * in + 16 * q;
  const uint16_t* xrow[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t)
    xrow[t] = x + static_cast<int64_t>(min(t0 + 16 * t + i, tokens - 1)) * in + 16 * q;
  v4f acc[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int c0 = wave; c0 < nchunk; c0 += kLinMmaWaves * kLinMmaChunks) {
    u32x4 a[kLinMmaChunks][2], b[TT][kLinMmaChunks][2];
#pragma unroll
    for (int u = 0; u < kLinMmaChunks; ++u) {
      const int64_t o = static_cast<int64_t>(min(c0 + u * kLinMmaWaves, nchunk - 1)) * 64;
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        b[t][u][0] = load16(xrow[t] + o);
        b[t][u][1] = load16(xrow[t] + o + 8);
      }
      a[u][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + o));
      a[u][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + o + 8));
    }
    __builtin_amdgcn_sched_barrier(0);   // every load above is issued before the math below
#pragma unroll
    for (int u = 0; u < kLinMmaChunks; ++u) {
      // a chunk past the end re-read the last one: zeros in both operands
      // (no branch, which would put each chunk's wait before the next
      // chunk's loads)
      const bool live = c0 + u * kLinMmaWaves < nchunk;
      const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        a[u][h] = live ? a[u][h] : z;
#pragma unroll
        for (int t = 0; t < TT; ++t) b[t][u][h] = live ? b[t][u][h] : z;
      }
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        acc[t] = mfma_bf16_16x16x32(a[u][0], b[t][u][0], acc[t]);
        acc[t] = mfma_bf16_16x16x32(a[u][1], b[t][u][1], acc[t]);
      }
    }
  }
  // lane (q, i) holds rows 4q .. 4q + 3 of token column i
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) part[wave][t][4 * q + r][i] = acc[t][r];
  __syncthreads();
  for (int o = threadIdx.x; o < TT * 256; o += 64 * kLinMmaWaves) {
    const int t = o >> 8, j = (o >> 4) & 15, rr = o & 15;
    float v = part[0][t][rr][j];
#pragma unroll
    for (int s = 1; s < kLinMmaWaves; ++s) v += part[s][t][rr][j];
    const int tok = t0 + 16 * t + j;
    if (tok < tokens) y[static_cast<int64_t>(tok) * out + r0 + rr] = f32_to_bf16(v);
  }
}

// Token tiles per workgroup: 1 up to 16 tokens, 2 up to 64, 4 beyond (W is
// read once per workgroup column).  Measured on MI355X ([2048, 2048], a
// graph over 40 layers' matrices): 5.0 / 5.3 / 6.0 / 7.7 / 7.7 / 11.2 us at
// 5 / 8 / 16 / 32 / 64 / 128 tokens, against 10.9 / 11.1 / 11.2 us for
// torch.mm (hipBLASLt) at 8 / 32 / 128; 16 waves per workgroup or 2 chunks
// in flight changed nothing below 32 tokens and lost above, 8 tiles per
// workgroup (W read once) took 19.2 us at 128.
static void launch_linear_mma(const uint16_t* x, const uint16_t* w, int32_t tokens, int32_t in,
                              int32_t out, uint16_t* y, hipStream_t s) {
  const dim3 block(64 * kLinMmaWaves);
  if (tokens <= 16)
    hipLaunchKernelGGL((linear_bf16_mma_kernel<1>), dim3(out / 16, 1), block, 0, s, x, w, tokens,
                       in, out, y);
  else if (tokens <= 64)
    hipLaunchKernelGGL((linear_bf16_mma_kernel<2>), dim3(out / 16, (tokens + 31) / 32), block, 0,
                       s, x, w, tokens, in, out, y);
  else
    hipLaunchKernelGGL((linear_bf16_mma_kernel<4>), dim3(out / 16, (tokens + 63) / 64), block, 0,
                       s, x, w, tokens, in, out, y);
}

template <int NR, bool ADD>
static void launch_linear(const uint16_t* x, const uint16_t* xa, const uint16_t* w,
                          int32_t tokens, int32_t in, int32_t out, uint16_t* y, hipStream_t s) {
  const unsigned grid = static_cast<unsigned>((out + kLinearWaves * NR - 1) / (kLinearWaves * NR));
  if (tokens == 1)
    hipLaunchKernelGGL((linear_bf16_kernel<NR, 1, ADD>), dim3(grid), dim3(64 * kLinearWaves), 0,
                       s, x, xa, w, tokens, in, out, y);
  else
    hipLaunchKernelGGL((linear_bf16_kernel<NR, kLinearMaxTokens, ADD>), dim3(grid),
                       dim3(64 * kLinearWaves), 0, s, x, xa, w, tokens, in, out, y);
}

template <int NR>
static void launch_linear(const uint16_t* x, const uint16_t* xa, const uint16_t* w,
                          int32_t tokens, int32_t in, int32_t out, uint16_t* y, hipStream_t s) {
  if (xa)
    launch_linear<NR, true>(x, xa, w, tokens, in, out, y, s);
  else
    launch_linear<NR, false>(x, xa, w, tokens, in, out, y, s);
}

}  // namespace moe

using namespace moe;

extern "C" int moe_linear_bf16(const void* x, const void* x_add, const void* w, int32_t tokens,
                               int32_t in_features, int32_t out_features, void* y,
                               int32_t rows_per_wave, void* stream) {
  MOE_REQUIRE(x && w && y, "moe_linear_bf16: NULL pointer");
  MOE_REQUIRE(tokens >= 1 && tokens <= kLinMmaMaxTokens,
              "moe_linear_bf16: need 1 <= tokens <= %d", kLinMmaMaxTokens);
  MOE_REQUIRE(tokens <= kLinearMaxTokens ||
                  (!x_add && in_features % 64 == 0 && out_features % 16 == 0),
              "moe_linear_bf16: beyond %d tokens, in_features must be a multiple of 64, "
              "out_features of 16, and x_add NULL", kLinearMaxTokens);
  MOE_REQUIRE(in_features >= 8 && in_features % 8 == 0 && out_features >= 1,
              "moe_linear_bf16: in_features must be a positive multiple of 8, out_features >= 1");
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(x_add) % 16 == 0,
              "moe_linear_bf16: x, x_add and w must be 16-byte aligned");
  MOE_REQUIRE(rows_per_wave == 0 || rows_per_wave == 1 || rows_per_wave == 2 || rows_per_wave == 4,
              "moe_linear_bf16: rows_per_wave must be 0 (default), 1, 2 or 4");
  hipStream_t s = as_stream(stream);
  const auto* xb = static_cast<const uint16_t*>(x);
  const auto* ab = static_cast<const uint16_t*>(x_add);
  const auto* wb = static_cast<const uint16_t*>(w);
  auto* yb = static_cast<uint16_t*>(y);
  if (tokens > kLinearMaxTokens) {
    launch_linear_mma(xb, wb, tokens, in_features, out_features, yb, s);
    return check_launch("moe_linear_bf16");
  }
  switch (rows_per_wave) {
    case 2: launch_linear<2>(xb, ab, wb, tokens, in_features, out_features, yb, s); break;
    case 4: launch_linear<4>(xb, ab, wb, tokens, in_features, out_features, yb, s); break;
    default: launch_linear<1>(xb, ab, wb, tokens, in_features, out_features, yb, s); break;
  }
  return check_launch("moe_linear_bf16");
}
