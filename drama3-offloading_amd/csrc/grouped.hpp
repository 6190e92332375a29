// Launchers shared between translation units of libmoeoffload.
#pragma once

#include "common.hpp"

namespace moe {

// The grouped path's activation rows: x [tokens, hidden] bf16 -> e4m3 codes
// xq and per-128 scales xs, one 256-thread slice per token (16 threads x 8
// values per 128-group).
struct QuantRowsJob {
  const uint16_t* x;
  int32_t hidden;
  uint8_t* xq;
  float* xs;
  int32_t tokens;
};

__device__ __forceinline__ void quant_row(const QuantRowsJob& q, int64_t t, int tid) {
  const uint16_t* xr = q.x + t * q.hidden;
  for (int base = 0; base < q.hidden; base += 2048) {
    const int i = base + tid * 8;
    float v[8];
    float amax = 0.0f;
    if (i < q.hidden) {
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
    amax = row16_max_f32(amax);
    if (i < q.hidden) {
      const float s = act_scale(amax);
      *reinterpret_cast<uint2*>(q.xq + t * q.hidden + i) =
          make_uint2(quant4_e4m3(v, s), quant4_e4m3(v + 4, s));
      if ((tid & 15) == 0) q.xs[t * (q.hidden >> 7) + (i >> 7)] = s;
    }
  }
}

// permute.hip
// tiles (nullable): (expert, first segment row) of every tile_tokens rows of
// every expert's segment, in expert order, and their count in *n_tiles.
// quant (nullable): activation rows quantised by extra workgroups of the
// same launch, two tokens each, beside the one that permutes.
int launch_permute(const void* ids, int ids64, int64_t P, int32_t n_experts, int32_t* counts,
                   int32_t* offsets, int32_t* sorted_pairs, int32_t* pair_pos, hipStream_t s,
                   int32_t* tiles = nullptr, int32_t* n_tiles = nullptr, int32_t tile_tokens = 16,
                   const QuantRowsJob* quant = nullptr);
int launch_unpermute(const float* y, const int32_t* pair_pos, const void* weights, int wbf16,
                     int32_t tokens, int32_t top_k, int32_t hidden, const uint16_t* residual,
                     uint16_t* out, hipStream_t s);

// grouped.hip: workspace layout of the grouped path (byte offsets, 256-aligned)
struct GroupedLayout {
  size_t counts, offsets, sorted, pos, tiles, n_tiles, xq, xs, h, aq, as, y, total;
};
GroupedLayout grouped_layout(int32_t tokens, int32_t top_k, int32_t n_experts, int32_t hidden,
                             int32_t inter);
int launch_grouped(const uint16_t* x, const void* ids, int ids64, const void* weights, int wbf16,
                   int32_t tokens, int32_t top_k, const uint8_t* w13, const float* s13,
                   const uint8_t* w2, const float* s2, const moe_expert_strides& es,
                   int32_t n_experts, int32_t hidden, int32_t inter, const uint16_t* residual,
                   uint16_t* out, char* ws, hipStream_t s);

}  // namespace moe
