// OCP e4m3fn encoder shared by every kernel, also compiled for the host so the
// CPU tests can check it against the oracle on every tie and boundary.
#pragma once

#include <math.h>
#include <stdint.h>

#if defined(__HIP__)
#define MOE_HOST_DEVICE __host__ __device__ __forceinline__
#else
#define MOE_HOST_DEVICE inline
#endif

namespace moe {

// float -> e4m3fn code, round-to-nearest-even, saturating at +-448, NaN -> 0x7f.
// Branch-free: every case is computed and the right one selected.
//   normal results (|v| >= 2^-6): round the 23-bit float mantissa to 3 bits
//     on the bit pattern (add 2^19 - 1 plus the kept LSB, shift by 20; a
//     carry moves into the exponent as it should), then rebias 127 -> 7;
//   subnormal results: |v| * 512 is exact and rintf rounds it to the 2^-9
//     grid (8 is the smallest normal, code 8, so the two ranges meet);
//   |v| >= 448 (including inf) saturates to 0x7e.
MOE_HOST_DEVICE uint32_t f32_to_e4m3(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t mag = u & 0x7fffffffu;
  const uint32_t normal = ((mag + 0x7ffffu + ((mag >> 20) & 1u)) >> 20) - (120u << 3);
  const uint32_t sub =
      static_cast<uint32_t>(rintf(__builtin_bit_cast(float, mag) * 512.0f));
  uint32_t code = mag < 0x3c800000u ? sub : normal;   // 2^-6
  code = mag >= 0x43e00000u ? 0x7eu : code;           // 448
  code = mag > 0x7f800000u ? 0x7fu : code;            // NaN
  return sign | code;
}

// Per-128-group activation scale: amax / 448 in float32, division correctly
// rounded.
MOE_HOST_DEVICE float act_scale(float amax) { return amax / 448.0f; }

// Quantise v with scale s: e4m3(v / s), the quotient correctly rounded to
// float32 first; s == 0 (an all-zero group) gives code 0.
MOE_HOST_DEVICE uint32_t quant_e4m3(float v, float s) {
  const uint32_t c = f32_to_e4m3(v / s);
  return s == 0.0f ? 0u : c;
}

#if defined(__HIP__)
// f32_to_e4m3 of four values, packed little-endian, on the conversion unit:
// v_cvt_pk_fp8_f32 (OCP e4m3, round to nearest even) of each value clamped
// to +-448 (beyond 448 the unclamped conversion gives NaN, the encoder
// saturates), NaN inputs given the encoder's sign | 0x7f.  Equal to four
// f32_to_e4m3 calls for every float input; moe_e4m3_check compares the two
// on the device over any range of bit patterns.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  const float v[4] = {a, b, c, d};
  float k[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) k[i] = __builtin_amdgcn_fmed3f(v[i], -448.0f, 448.0f);
  uint32_t w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(k[0], k[1], 0, false));
  w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(k[2], k[3], static_cast<int>(w), true));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (v[i] != v[i]) {
      const uint32_t nan = ((__builtin_bit_cast(uint32_t, v[i]) >> 24) & 0x80u) | 0x7fu;
      w = (w & ~(0xffu << (8 * i))) | (nan << (8 * i));
    }
  }
  return w;
}

// quant_e4m3 of v[0..3] with one scale, packed little-endian.
__device__ __forceinline__ uint32_t quant4_e4m3(const float* v, float s) {
  const uint32_t w = e4m3x4(v[0] / s, v[1] / s, v[2] / s, v[3] / s);
  return s == 0.0f ? 0u : w;
}
#endif

}  // namespace moe
