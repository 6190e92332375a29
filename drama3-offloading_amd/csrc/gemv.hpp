// The decode GEMV's down launch, for a caller that forms the SiLU(gate) * up
// rows itself (the decode step's fused launch in decode_step.hip).
#pragma once

#include "common.hpp"

namespace moe {

// The MoE block's shared expert carried along by the two decode launches
// (moe_fp8_moe_block_forward): kernel 1 computes its act and sigmoid gate in
// extra workgroups, kernel 2 its down rows in one extra wave per workgroup,
// with the arithmetic of the standalone shared-expert kernels (shared.hpp).
struct SharedRefs {
  const uint16_t* wg;    // [Is, H] bf16
  const uint16_t* wu;    // [Is, H]
  const uint16_t* wd;    // [H, Is]
  const uint16_t* wsg;   // [H]
  int32_t inter;         // Is
  uint16_t* act;         // [T, Is] bf16 scratch
  float* sig;            // [T] scratch
};
constexpr int kSharedJPW = 2;   // shared intermediate rows (gate + up) per kernel-1 wave

// A slot table's next state, staged by the launch that resolved the call
// (its workgroups all read the table, so none of them may write it), and
// copied into the table by one extra workgroup of the down launch, which
// reads no table.  n_experts == 0: nothing to copy.
struct TableCommit {
  const int32_t* so_src;
  int32_t* so_dst;
  const int32_t* se_src;
  int32_t* se_dst;
  const int64_t* st_src;
  int64_t* st_dst;
  const int64_t* step_src;
  int64_t* step_dst;
  int32_t n_experts;
  int32_t cap;
};

// Limits of the decode GEMV kernels.
constexpr int kGemvMaxHidden = 8192;
constexpr int kGemvMaxInter = 2048;
constexpr int kGemvMaxTopK = 16;

// down_gemv_kernel over `tokens` tokens of top_k pairs each: out[t] =
// bf16(residual[t] + bf16(sum_k fma-in-order weights[t,k] * y_k)) (no
// residual: the bf16 sum), y_k = W2[slots[t,k]] . quantised act[t*top_k+k];
// act [pairs, inter] f32, slots int32, weights f32 (bf16 when wbf16); w2 /
// s2 with expert strides w2_es bytes / s2_es floats, tile order when `tiled`.  With `sh`,
// the shared expert's down rows ride along (its act and sig formed before)
// and out = residual + (routed + sig * shared), as the block call gives.
// With `commit` (nullable), one more workgroup copies a staged slot table
// into the table.  Launch errors are returned (check_launch).
int launch_down_gemv(const float* act, const int32_t* slots, const void* weights, int wbf16,
                     int32_t tokens, int32_t top_k, const uint8_t* w2, const float* s2,
                     int64_t w2_es, int64_t s2_es, int tiled, int32_t n_slots, int32_t hidden,
                     int32_t inter, const uint16_t* residual, uint16_t* out,
                     const SharedRefs* sh, hipStream_t s, const TableCommit* commit = nullptr);

}  // namespace moe
