// The arithmetic of the shared expert, used by its own kernels (shared.hip)
// and by the decode GEMV kernels that carry it along (moe_gemv.hip), so that
// both give bit-identical results.
#pragma once

#include "common.hpp"

namespace moe {

__device__ __forceinline__ u32x4 load16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// acc + sum of the 8 bf16 products of two 16-byte slices, one fma each in order.
__device__ __forceinline__ float dot8_bf16(u32x4 w, u32x4 x, float acc) {
  const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
  const uint32_t xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc = fmaf(__uint_as_float(wv[i] << 16), __uint_as_float(xv[i] << 16), acc);
    acc = fmaf(__uint_as_float(wv[i] & 0xffff0000u), __uint_as_float(xv[i] & 0xffff0000u), acc);
  }
  return acc;
}

// The 64 lane sums added: DPP within rows of 16 lanes, then the four rows in
// order (no LDS round trips, which a shuffle butterfly takes six of).
__device__ __forceinline__ float wave_sum_f32(float v) { return wave_sum_f32_dpp(v); }

// bf16 rounding of an f32 value, returned as f32.
__device__ __forceinline__ float rbf16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// acc[i][t] = <row_i, x[t0 + t]> over n16 16-byte slices (8 bf16 each), the
// one dot product every shared-expert product uses: lane l sums slices
// l, l + 64, l + 128, ... in that order with one fma per product, then the 64
// lane sums are added by wave_sum_f32 (every lane ends with the total).  U
// slices per lane are loaded before any is used; slices past the end load
// the last slice again and are not summed.  Tokens past `tokens` repeat the
// last token.  U changes only the load schedule, never the sums.
template <int NR, int TB, int U>
__device__ __forceinline__ void rows_dot_bf16(const uint16_t* const (&rows)[NR],
                                              const uint16_t* __restrict__ x, int64_t x_stride,
                                              int t0, int tokens, int n16, int lane,
                                              float (&acc)[NR][TB]) {
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int t = 0; t < TB; ++t) acc[i][t] = 0.0f;
  for (int c0 = 0; c0 < n16; c0 += 64 * U) {
    u32x4 w[U][NR], xv[TB][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(c0 + u * 64 + lane, n16 - 1);
#pragma unroll
      for (int i = 0; i < NR; ++i) w[u][i] = load16(rows[i] + c * 8);
    }
#pragma unroll
    for (int t = 0; t < TB; ++t)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = min(c0 + u * 64 + lane, n16 - 1);
        xv[t][u] = load16(x + static_cast<int64_t>(min(t0 + t, tokens - 1)) * x_stride + c * 8);
      }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (c0 + u * 64 + lane >= n16) continue;
#pragma unroll
      for (int t = 0; t < TB; ++t)
#pragma unroll
        for (int i = 0; i < NR; ++i) acc[i][t] = dot8_bf16(w[u][i], xv[t][u], acc[i][t]);
    }
  }
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int t = 0; t < TB; ++t) acc[i][t] = wave_sum_f32(acc[i][t]);
}

// act = bf16(bf16(silu(bf16(g))) * bf16(u)) from the gate and up row sums.
__device__ __forceinline__ uint16_t shared_act(float gsum, float usum) {
  const float g = rbf16(gsum);
  const float u = rbf16(usum);
  const float s = rbf16(g / (1.0f + expf(-g)));
  return f32_to_bf16(s * u);
}

// bf16(sigmoid(bf16(z))) from the gate row's sum, as an f32 value.
__device__ __forceinline__ float shared_sig(float zsum) {
  const float z = rbf16(zsum);
  return rbf16(1.0f / (1.0f + expf(-z)));
}

// bf16(sig * bf16(d)), then + routed and + residual (each when present),
// each rounded to bf16.  The callers load routed and residual early: they do
// not depend on the sums, and a load after them would add a memory round trip.
__device__ __forceinline__ uint16_t shared_out(float dsum, float sig, bool has_routed,
                                               uint16_t routed, bool has_residual,
                                               uint16_t residual) {
  float v = rbf16(sig * rbf16(dsum));
  if (has_routed) v = rbf16(bf16_to_f32(routed) + v);
  if (has_residual) v = rbf16(bf16_to_f32(residual) + v);
  return f32_to_bf16(v);
}

// Launchers of the standalone shared-expert kernels (shared.hip).
int launch_shared_gate_up(const uint16_t* x, const uint16_t* wg, const uint16_t* wu,
                          const uint16_t* wsg, int32_t tokens, int32_t hidden, int32_t inter,
                          uint16_t* act, float* sig, hipStream_t s);
int launch_shared_down(const uint16_t* act, const float* sig, const uint16_t* wd, int32_t tokens,
                       int32_t hidden, int32_t inter, const uint16_t* routed,
                       const uint16_t* residual, uint16_t* out, hipStream_t s);

}  // namespace moe
