// Launchers shared between translation units of libmoeoffload.
#pragma once

#include "common.hpp"

namespace moe {

// permute.hip
// tiles (nullable): (expert, first segment row) of every tile_tokens rows of
// every expert's segment, in expert order, and their count in *n_tiles.
int launch_permute(const void* ids, int ids64, int64_t P, int32_t n_experts, int32_t* counts,
                   int32_t* offsets, int32_t* sorted_pairs, int32_t* pair_pos, hipStream_t s,
                   int32_t* tiles = nullptr, int32_t* n_tiles = nullptr, int32_t tile_tokens = 16);
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
