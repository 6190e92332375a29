// Shared helpers for libmoeoffload: error reporting, launch checks, bf16 and
// e4m3fn arithmetic used identically by every kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/moe_offload.h"
#include "e4m3.hpp"

namespace moe {

// Thread-local text of the last failure; set by fail()/check_launch().
void set_error(const char* fmt, ...);
void clear_error();

#define MOE_REQUIRE(cond, ...)        \
  do {                                \
    if (!(cond)) {                    \
      ::moe::set_error(__VA_ARGS__);  \
      return MOE_EINVAL;              \
    }                                 \
  } while (0)

// Sync-free launch check: reads the sticky launch error without waiting.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ----------------------------------------------------------------- bf16

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even float -> bf16 bits (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// SiLU(g) * u in float32, the one formula every expert kernel uses:
// g * rcp(1 + 2^(-g log2 e)) * u on the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32).  The rounded argument -g log2 e puts about
// 0.7 |g| * 2^-24 of relative error into exp2, and the hardware exp2 adds
// more at large arguments: measured against float64 on a dense grid of
// |g| <= 40, the result is within (2 |g| + 8) * 2^-24 relative of
// SiLU(g) * u (moe_silu_check), against an e4m3 step of 2^-3 once
// quantised.  An IEEE division and the library expf cost about 25 more
// VALU instructions per value, on the critical path of the decode down
// kernel.
// g past -88 gives exp2 = inf, rcp = 0 and -0 (as g / inf); NaN propagates.
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// ------------------------------------------------------------ wave utils
//
// The DPP exchanges below (quad permutes and row mirrors) read only lanes
// inside the reading lane's row of 16, so the bound control never applies;
// they are written with old = 0 and bound_ctrl set, the form the compiler
// folds into the instruction that consumes the exchange (v_max_u32_dpp,
// v_add_f32_dpp) instead of a separate copy and DPP move.  An inactive
// source lane would read as 0 in this form, so every lane of a row of 16
// (of the wave, for the wave-wide reductions) takes part in each call.

// Max over each row of 16 lanes, in every lane of the row, by DPP exchanges
// (quad xor 1, quad xor 2, half-row mirror, row mirror): no LDS crossbar, so
// no wait on the counter that LDS and scalar loads share.  fmaxf ignores a
// NaN operand in any order, so this equals a shuffle butterfly bit for bit.
__device__ __forceinline__ float row16_max_f32(float v) {
#define MOE_DPP_MAX(CTRL)                                                                  \
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, \
                                                          true)));
  MOE_DPP_MAX(0x0B1)   // quad_perm [1,0,3,2]
  MOE_DPP_MAX(0x04E)   // quad_perm [2,3,0,1]
  MOE_DPP_MAX(0x141)   // row_half_mirror
  MOE_DPP_MAX(0x140)   // row_mirror
#undef MOE_DPP_MAX
  return v;
}

// SiLU(gate) * up of 8 intermediate columns j..j+7 held by one lane
// (hr = gate[j..j+3], gate[j+4..j+7], up[j..j+3], up[j+4..j+7]) -> e4m3
// codes and the group scale in LDS; 16 consecutive lanes form one 128-group.
// Every lane of the wave calls this, lanes past the end with live == false.
__device__ __forceinline__ void silu_quantize8(const float4 (&hr)[4], bool live, int j,
                                               uint8_t* __restrict__ aq, float* __restrict__ as) {
  const float gv[8] = {hr[0].x, hr[0].y, hr[0].z, hr[0].w, hr[1].x, hr[1].y, hr[1].z, hr[1].w};
  const float uv[8] = {hr[2].x, hr[2].y, hr[2].z, hr[2].w, hr[3].x, hr[3].y, hr[3].z, hr[3].w};
  float av[8];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    av[i] = silu_mul(gv[i], uv[i]);
    amax = fmaxf(amax, fabsf(av[i]));
  }
  amax = row16_max_f32(amax);
  if (live) {
    const float sc = act_scale(amax);
    *reinterpret_cast<uint2*>(aq + j) = make_uint2(quant4_e4m3(av, sc), quant4_e4m3(av + 4, sc));
    if ((threadIdx.x & 15) == 0) as[j >> 7] = sc;
  }
}


// 8 bf16 values of x held by one lane (16 bytes, elements i..i+7) -> e4m3
// codes and the group scale in LDS.  Sixteen consecutive lanes form one
// 128-column group; every lane of the wave calls this (the group maximum is
// a cross-lane exchange), lanes past the end with live == false.
__device__ __forceinline__ void quantize_x8(uint4 raw, bool live, int i,
                                            uint8_t* __restrict__ xq, float* __restrict__ xs) {
  const uint32_t rr[4] = {raw.x, raw.y, raw.z, raw.w};
  float v[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = __uint_as_float(rr[j] << 16);
    v[2 * j + 1] = __uint_as_float(rr[j] & 0xffff0000u);
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
  amax = row16_max_f32(amax);
  if (live) {
    const float sc = act_scale(amax);
    *reinterpret_cast<uint2*>(xq + i) = make_uint2(quant4_e4m3(v, sc), quant4_e4m3(v + 4, sc));
    if ((threadIdx.x & 15) == 0) xs[i >> 7] = sc;
  }
}

// 8 float32 activations j..j+7 held by one lane -> e4m3 codes and the group
// scale in LDS; 16 consecutive lanes form one 128-group.
__device__ __forceinline__ void quantize8_f32(const float4 (&vr)[2], bool live, int j,
                                              uint8_t* __restrict__ aq, float* __restrict__ as) {
  const float av[8] = {vr[0].x, vr[0].y, vr[0].z, vr[0].w, vr[1].x, vr[1].y, vr[1].z, vr[1].w};
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(av[i]));
  amax = row16_max_f32(amax);
  if (live) {
    const float sc = act_scale(amax);
    *reinterpret_cast<uint2*>(aq + j) = make_uint2(quant4_e4m3(av, sc), quant4_e4m3(av + 4, sc));
    if ((threadIdx.x & 15) == 0) as[j >> 7] = sc;
  }
}

template <typename T>
__device__ __forceinline__ T wave_bcast(T v, int lane) { return __shfl(v, lane, 64); }

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Wave-wide maximum of a 32-bit unsigned value, returned as a scalar: the
// row-of-16 DPP exchanges of wave_reduce_u64 on one register, then the
// four row maxima combined on the scalar unit.  About a third of the
// 64-bit reduction's instructions.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#define MOE_DPP_UMAX(CTRL)                                                             \
  {                                                                                    \
    const uint32_t o = __builtin_amdgcn_update_dpp(0u, v, CTRL, 0xf, 0xf, true);       \
    v = o > v ? o : v;                                                                 \
  }
  MOE_DPP_UMAX(0x0B1)   // quad_perm [1,0,3,2]
  MOE_DPP_UMAX(0x04E)   // quad_perm [2,3,0,1]
  MOE_DPP_UMAX(0x141)   // row_half_mirror
  MOE_DPP_UMAX(0x140)   // row_mirror
#undef MOE_DPP_UMAX
  const uint32_t a = __builtin_amdgcn_readlane(static_cast<int>(v), 0);
  const uint32_t b = __builtin_amdgcn_readlane(static_cast<int>(v), 16);
  const uint32_t c = __builtin_amdgcn_readlane(static_cast<int>(v), 32);
  const uint32_t d = __builtin_amdgcn_readlane(static_cast<int>(v), 48);
  const uint32_t ab = a > b ? a : b, cd = c > d ? c : d;
  return ab > cd ? ab : cd;
}

// Wave-wide max / min of a 64-bit key, returned uniform (in every lane):
// DPP exchanges inside each row of 16 lanes (quad xor 1, quad xor 2, half-row
// mirror, row mirror), then the four row results are read as scalars.  A
// handful of VALU cycles per step instead of an LDS-crossbar shuffle.
template <bool kMax>
__device__ __forceinline__ uint64_t wave_reduce_u64(uint64_t v) {
  uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
#define MOE_DPP_STEP(CTRL)                                                             \
  {                                                                                    \
    const uint32_t olo = __builtin_amdgcn_update_dpp(0u, lo, CTRL, 0xf, 0xf, true);    \
    const uint32_t ohi = __builtin_amdgcn_update_dpp(0u, hi, CTRL, 0xf, 0xf, true);    \
    const uint64_t o = (static_cast<uint64_t>(ohi) << 32) | olo;                       \
    const uint64_t c = (static_cast<uint64_t>(hi) << 32) | lo;                         \
    if (kMax ? (o > c) : (o < c)) {                                                    \
      lo = olo;                                                                        \
      hi = ohi;                                                                        \
    }                                                                                  \
  }
  MOE_DPP_STEP(0x0B1)   // quad_perm [1,0,3,2]
  MOE_DPP_STEP(0x04E)   // quad_perm [2,3,0,1]
  MOE_DPP_STEP(0x141)   // row_half_mirror
  MOE_DPP_STEP(0x140)   // row_mirror
#undef MOE_DPP_STEP
  uint64_t best = 0;
#pragma unroll
  for (int row = 0; row < 4; ++row) {
    const uint64_t x =
        (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(hi), row * 16))) << 32) |
        static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(lo), row * 16));
    best = row == 0 ? x : (kMax ? (x > best ? x : best) : (x < best ? x : best));
  }
  return best;
}

// Sum over the wave, uniform in every lane: DPP butterfly within each row of
// 16 lanes, then the four row sums read as scalars and added in row order.
__device__ __forceinline__ float wave_sum_f32_dpp(float v) {
#define MOE_DPP_ADD(CTRL)                                                                  \
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
  MOE_DPP_ADD(0x0B1)   // quad_perm [1,0,3,2]
  MOE_DPP_ADD(0x04E)   // quad_perm [2,3,0,1]
  MOE_DPP_ADD(0x141)   // row_half_mirror
  MOE_DPP_ADD(0x140)   // row_mirror
#undef MOE_DPP_ADD
  float s = 0.0f;
#pragma unroll
  for (int row = 0; row < 4; ++row)
    s += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), row * 16));
  return s;
}

// Value of lane `src` (uniform) as a scalar.
__device__ __forceinline__ int32_t lane_value(int32_t v, int src) {
  return __builtin_amdgcn_readlane(v, src);
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ---------------------------------------------------------------- MFMA

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 32 bytes (two 16-byte loads) as an MFMA operand; `p` 16-byte aligned.
__device__ __forceinline__ v8i load_op32(const uint8_t* p) {
  const u32x4* s = reinterpret_cast<const u32x4*>(p);
  u32x4 lo = s[0];
  u32x4 hi = s[1];
  return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

// Where a lane finds its MFMA A operand in an expert's [R, K] e4m3 weight
// matrix: the 32 bytes of row `row`, reduction indices [32q, 32q + 32) of
// K-block 0, as two 16-byte halves `half` bytes apart; K-block b is b *
// `kstep` further on, and the row 16 below is 16 * K further on in both
// orders.
//   row-major:   row * K + 32q;                          kstep 128,  half 16
//   MFMA tiles:  (row & ~15) * K + (16q + row % 16) * 16; kstep 2048, half 1024
// In tile order the 64 lanes of a wave loading rows 16g..16g+15 read 1 KiB
// contiguous per 16-byte load (8 whole 128-byte lines); row-major, the same
// load touches 16 lines, half of each.  The bytes each lane receives are
// the same, so are the products.
struct OperandWalk {
  int64_t off;
  int32_t kstep;
  int32_t half;
};
__device__ __forceinline__ OperandWalk operand_walk(int row, int q, int64_t K, bool tiled) {
  if (tiled)
    return {static_cast<int64_t>(row & ~15) * K + (16 * q + (row & 15)) * 16, 2048, 1024};
  return {static_cast<int64_t>(row) * K + 32 * q, 128, 16};
}
// The weight operand: nontemporal, streamed from HBM without keeping the
// lines in the caches.
__device__ __forceinline__ v8i load_op_nt(const uint8_t* p, int half) {
  u32x4 lo = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  u32x4 hi = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + half));
  return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

// acc += d * sc with one fused multiply-add (one rounding) per element,
// written out so that every kernel rounds its block sums identically.
__device__ __forceinline__ void block_fma(v4f& acc, const v4f& d, float sc) {
  acc[0] = fmaf(d[0], sc, acc[0]);
  acc[1] = fmaf(d[1], sc, acc[1]);
  acc[2] = fmaf(d[2], sc, acc[2]);
  acc[3] = fmaf(d[3], sc, acc[3]);
}

// 16x16x128 e4m3 x e4m3 -> f32 on gfx950, block scales neutral (E8M0 127 = 1.0).
// Lane l supplies row (l % 16) of A and column (l % 16) of B, 32 bytes each,
// covering the same 32 reduction indices for both operands; the four lane
// groups (l / 16) cover disjoint 32-index sets, so the product is the full
// 128-term dot product.  Result: lane l holds C[4*(l/16) + i][l % 16].
__device__ __forceinline__ v4f mfma_e4m3_16x16x128(v8i a, v8i b, v4f c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

}  // namespace moe
