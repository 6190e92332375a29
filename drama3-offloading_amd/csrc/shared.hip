// Shared expert of the MoE block (bf16, dense, every token) and the decode
// step's finiteness guard.
//
// The MoE block's output with a gated shared expert, in the bf16 op order of
// the model's own modules (every Linear rounds its f32 sum to bf16, every
// elementwise op rounds its f32 result to bf16):
//
//   g, u  = x W_gate^T, x W_up^T                  [T, Is]
//   a     = bf16(silu(g)) * u                      [T, Is]
//   d     = a W_down^T                             [T, H]
//   s     = bf16(sigmoid(x w_sg^T))                [T, 1]
//   out   = residual + (routed + s * d)            [T, H]
//
// moe_shared_gate_up computes a and s (one wave per intermediate row j,
// holding the gate and up rows of j; one extra wave for the sigmoid gate
// row), moe_shared_down the rest (4 output rows per wave) with the routed
// output and the residual added in its epilogue.  Both are GEMVs over
// weights read once per 4 tokens (per token at decode): HBM-bound, 6 MiB per
// layer at H = 2048, Is = 512.  Sums are f32 fused multiply-adds over each
// lane's 16-byte slices in row order, then the 64 lane sums (wave_sum_f32).
#include "shared.hpp"

namespace moe {

constexpr int kSharedTB = 4;   // tokens per pass over the weights (1 when there is one)
constexpr int kUnroll = 4;     // 16-byte slices per lane in flight per row
// Waves per workgroup: small workgroups spread the rows over every CU.  A
// 1-token call (both kernels, 2048 x 512) measured 7.07 us at 2, 7.12 at 1
// and 7.47 at 4 on MI355X.
constexpr int kWavesPerWG = 2;

template <int TB>
__global__ __launch_bounds__(64 * kWavesPerWG) void shared_gate_up_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg, const uint16_t* __restrict__ wu,
    const uint16_t* __restrict__ wsg, int32_t tokens, int32_t hidden, int32_t inter,
    uint16_t* __restrict__ act, float* __restrict__ sig) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int j = blockIdx.x * kWavesPerWG + wave; // j == inter: the sigmoid gate row
  if (j > inter) return;                         // no barriers below
  const bool gate_row = j == inter;
  const uint16_t* const rows[2] = {gate_row ? wsg : wg + static_cast<int64_t>(j) * hidden,
                                   gate_row ? wsg : wu + static_cast<int64_t>(j) * hidden};
  for (int t0 = 0; t0 < tokens; t0 += TB) {
    float acc[2][TB];
    rows_dot_bf16<2, TB, kUnroll>(rows, x, hidden, t0, tokens, hidden >> 3, lane, acc);
    if (lane == 0) {
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        if (t0 + t >= tokens) break;
        if (gate_row)
          sig[t0 + t] = shared_sig(acc[0][t]);
        else
          act[static_cast<int64_t>(t0 + t) * inter + j] = shared_act(acc[0][t], acc[1][t]);
      }
    }
  }
}

template <int TB, int U>
__global__ __launch_bounds__(64 * kWavesPerWG) void shared_down_kernel(
    const uint16_t* __restrict__ act, const float* __restrict__ sig,
    const uint16_t* __restrict__ wd, int32_t tokens, int32_t hidden, int32_t inter,
    const uint16_t* __restrict__ routed, const uint16_t* __restrict__ residual,
    uint16_t* __restrict__ out) {
  constexpr int kRows = 4;                        // output rows per wave
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r0 = (blockIdx.x * kWavesPerWG + wave) * kRows;
  if (r0 >= hidden) return;                       // hidden % 16 == 0: all kRows rows exist
  const uint16_t* rows[kRows];
#pragma unroll
  for (int i = 0; i < kRows; ++i) rows[i] = wd + static_cast<int64_t>(r0 + i) * inter;
  for (int t0 = 0; t0 < tokens; t0 += TB) {
    // lane i * TB + t finishes (row r0 + i, token t0 + t): its routed and
    // residual values and the token's gate go out before the weights (lanes
    // past the outputs re-read the last output's; an absent buffer reads the
    // first word of act, which the sums read anyway, and is ignored)
    const int li = min(lane, kRows * TB - 1);
    const int tt = min(t0 + li % TB, tokens - 1);
    const int64_t oo = static_cast<int64_t>(tt) * hidden + r0 + li / TB;
    const uint16_t rv = *(routed ? routed + oo : act);
    const uint16_t sv = *(residual ? residual + oo : act);
    const float sg = sig[tt];
    float acc[kRows][TB];
    rows_dot_bf16<kRows, TB, U>(rows, act, inter, t0, tokens, inter >> 3, lane, acc);
#pragma unroll
    for (int i = 0; i < kRows; ++i)
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        if (lane != i * TB + t || t0 + t >= tokens) continue;
        out[oo] = shared_out(acc[i][t], sg, routed != nullptr, rv, residual != nullptr, sv);
      }
  }
}

// flag = 1 when every element of x is finite, else 0.  One workgroup, so the
// flag is written exactly once and needs no clearing before (a graph replays
// it as is).
__global__ __launch_bounds__(1024) void all_finite_kernel(const void* __restrict__ x, int f32,
                                                          int64_t n, int32_t* __restrict__ flag) {
  bool ok = true;
  const int64_t nbytes = n * (f32 ? 4 : 2);
  const int64_t nvec = nbytes >> 4;               // whole 16-byte units
  const u32x4* v = reinterpret_cast<const u32x4*>(x);
  for (int64_t i = threadIdx.x; i < nvec; i += blockDim.x) {
    const u32x4 u = v[i];
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // all exponent bits set: Inf or NaN (f32: one value per word, bf16: two)
      ok = ok && (w[k] & 0x7f800000u) != 0x7f800000u && (f32 || (w[k] & 0x7f80u) != 0x7f80u);
    }
  }
  // the tail past the last whole unit, one element per thread
  const int64_t done = (nvec << 4) / (f32 ? 4 : 2);
  for (int64_t i = done + threadIdx.x; i < n; i += blockDim.x) {
    if (f32) {
      ok = ok && (reinterpret_cast<const uint32_t*>(x)[i] & 0x7f800000u) != 0x7f800000u;
    } else {
      ok = ok && (reinterpret_cast<const uint16_t*>(x)[i] & 0x7f80u) != 0x7f80u;
    }
  }
  const int all = __syncthreads_and(ok ? 1 : 0);
  if (threadIdx.x == 0) *flag = all ? 1 : 0;
}

int launch_shared_gate_up(const uint16_t* x, const uint16_t* wg, const uint16_t* wu,
                          const uint16_t* wsg, int32_t tokens, int32_t hidden, int32_t inter,
                          uint16_t* act, float* sig, hipStream_t s) {
  const unsigned grid = static_cast<unsigned>((inter + 1 + kWavesPerWG - 1) / kWavesPerWG);
  auto kern = tokens == 1 ? shared_gate_up_kernel<1> : shared_gate_up_kernel<kSharedTB>;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * kWavesPerWG), 0, s, x, wg, wu, wsg, tokens,
                     hidden, inter, act, sig);
  return check_launch("moe_shared_gate_up");
}

int launch_shared_down(const uint16_t* act, const float* sig, const uint16_t* wd, int32_t tokens,
                       int32_t hidden, int32_t inter, const uint16_t* routed,
                       const uint16_t* residual, uint16_t* out, hipStream_t s) {
  // one 16-byte slice per lane and row covers inter <= 512: no batch to fill
  const bool one = inter <= 512;
  auto kern = tokens == 1 ? (one ? shared_down_kernel<1, 1> : shared_down_kernel<1, kUnroll>)
                          : (one ? shared_down_kernel<kSharedTB, 1>
                                 : shared_down_kernel<kSharedTB, kUnroll>);
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(hidden / (4 * kWavesPerWG))),
                     dim3(64 * kWavesPerWG), 0, s, act, sig, wd, tokens, hidden, inter, routed,
                     residual, out);
  return check_launch("moe_shared_down");
}

}  // namespace moe

using namespace moe;

extern "C" int moe_shared_gate_up(const void* x, const void* w_gate, const void* w_up,
                                  const void* w_sgate, int32_t tokens, int32_t hidden,
                                  int32_t inter, void* act, float* sig, void* stream) {
  MOE_REQUIRE(tokens >= 0, "moe_shared_gate_up: tokens < 0");
  MOE_REQUIRE(hidden >= 128 && hidden % 128 == 0 && inter >= 128 && inter % 128 == 0,
              "moe_shared_gate_up: hidden and inter must be positive multiples of 128");
  if (tokens == 0) return MOE_OK;
  MOE_REQUIRE(x && w_gate && w_up && w_sgate && act && sig, "moe_shared_gate_up: NULL pointer");
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(w_gate) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(w_up) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(w_sgate) % 16 == 0,
              "moe_shared_gate_up: x and weights must be 16-byte aligned");
  return launch_shared_gate_up(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w_gate),
                               static_cast<const uint16_t*>(w_up),
                               static_cast<const uint16_t*>(w_sgate), tokens, hidden, inter,
                               static_cast<uint16_t*>(act), sig, as_stream(stream));
}

extern "C" int moe_shared_down(const void* act, const float* sig, const void* w_down,
                               int32_t tokens, int32_t hidden, int32_t inter, const void* routed,
                               const void* residual, void* out, void* stream) {
  MOE_REQUIRE(tokens >= 0, "moe_shared_down: tokens < 0");
  MOE_REQUIRE(hidden >= 128 && hidden % 128 == 0 && inter >= 128 && inter % 128 == 0,
              "moe_shared_down: hidden and inter must be positive multiples of 128");
  if (tokens == 0) return MOE_OK;
  MOE_REQUIRE(act && sig && w_down && out, "moe_shared_down: NULL pointer");
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(act) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(w_down) % 16 == 0,
              "moe_shared_down: act and w_down must be 16-byte aligned");
  return launch_shared_down(static_cast<const uint16_t*>(act), sig,
                            static_cast<const uint16_t*>(w_down), tokens, hidden, inter,
                            static_cast<const uint16_t*>(routed),
                            static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(out),
                            as_stream(stream));
}

extern "C" int moe_all_finite(const void* x, int32_t dtype, int64_t n, int32_t* flag,
                              void* stream) {
  MOE_REQUIRE(dtype == MOE_F32 || dtype == MOE_BF16, "moe_all_finite: dtype must be F32 or BF16");
  MOE_REQUIRE(n >= 0 && flag, "moe_all_finite: need n >= 0 and a flag");
  MOE_REQUIRE(n == 0 || x, "moe_all_finite: NULL x");
  MOE_REQUIRE(n == 0 || reinterpret_cast<uintptr_t>(x) % 16 == 0,
              "moe_all_finite: x must be 16-byte aligned");
  hipLaunchKernelGGL(all_finite_kernel, dim3(1), dim3(1024), 0, as_stream(stream), x,
                     dtype == MOE_F32 ? 1 : 0, n, flag);
  return check_launch("moe_all_finite");
}
