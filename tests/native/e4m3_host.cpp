// Host build of the kernels' e4m3 encoder (the very header the HIP kernels
// include), exported for the CPU tests.
#include <stddef.h>
#include <stdint.h>

#include "../../drama3-offloading_amd/csrc/e4m3.hpp"

extern "C" void encode_many(const float* v, uint8_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = static_cast<uint8_t>(moe::f32_to_e4m3(v[i]));
}

// codes for every positive float with bit pattern in [lo, hi)
extern "C" void encode_range(uint32_t lo, uint32_t hi, uint8_t* out) {
  for (uint32_t u = lo; u < hi; ++u)
    out[u - lo] = static_cast<uint8_t>(moe::f32_to_e4m3(__builtin_bit_cast(float, u)));
}

extern "C" void quant_many(const float* v, const float* s, uint8_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = static_cast<uint8_t>(moe::quant_e4m3(v[i], s[i]));
}
