// Top-k-of-E router: logits = x . W^T (+ bias), top-k by descending logit
// (ties to the lower expert), softmax over the k selected (== softmax over all
// E then renormalise, upstream's norm_topk_prob).
//
// Logit arithmetic: a bf16 x bf16 product is exact in float32; products are
// summed in float64 and rounded once to float32.  With float64 partial sums
// exact for ordinary data, the rounded logit does not depend on the order of
// summation, which is what lets expert ids match the oracle bit for bit.
//
// One launch: grid (E/4, ceil(T/4)), 4 waves per workgroup.  Wave w of
// workgroup (bx, by) computes the logit of expert 4*bx + w for the 4 tokens
// of token block `by`, reading its 4 KiB gate row once.  Each workgroup then
// bumps the token block's arrival counter; the last one to arrive selects the
// top-k of those tokens (one wave per token, logits in registers) and puts
// the counter back to zero, so the counters never need clearing between
// calls (nothing to memset inside a graph).
#include "common.hpp"

namespace moe {

constexpr int kMaxTopK = 32;
constexpr int kTokBlock = 4;

template <int PER>
__device__ void topk_one_token(const float* __restrict__ row, int32_t n_experts, int32_t top_k,
                               int64_t t, void* __restrict__ ids, int ids64,
                               void* __restrict__ weights, int wbf16) {
  const int lane = threadIdx.x & 63;
  float v[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = lane + 64 * j;
    // coherent loads: other workgroups wrote these logits
    v[j] = e < n_experts ? __hip_atomic_load(row + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                         : -INFINITY;
  }
  uint64_t taken = 0;   // bit j: expert lane + 64*j already selected
  float m = 0.0f, sum = 0.0f;
  float myv = 0.0f;
  int myi = 0;
  for (int r = 0; r < top_k; ++r) {
    float bv = 0.0f;
    int bi = INT32_MAX;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = lane + 64 * j;
      if (e < n_experts && !((taken >> j) & 1ull) && (bi == INT32_MAX || v[j] > bv)) {
        bv = v[j];
        bi = e;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (oi != INT32_MAX && (bi == INT32_MAX || ov > bv || (ov == bv && oi < bi))) {
        bv = ov;
        bi = oi;
      }
    }
    if ((bi & 63) == lane) taken |= 1ull << (bi >> 6);
    if (r == 0) m = bv;
    const float ex = expf(bv - m);
    sum += ex;
    if (lane == r) {       // lane r keeps round r's pick
      myv = ex;
      myi = bi;
    }
  }
  if (lane < top_k) {
    const int64_t o = t * top_k + lane;
    if (ids64) reinterpret_cast<int64_t*>(ids)[o] = myi;
    else reinterpret_cast<int32_t*>(ids)[o] = myi;
    const float wv = myv / sum;
    if (wbf16) reinterpret_cast<uint16_t*>(weights)[o] = f32_to_bf16(wv);
    else reinterpret_cast<float*>(weights)[o] = wv;
  }
}

template <int PER>
__global__ __launch_bounds__(256) void router_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const float* __restrict__ bias,
    int32_t tokens, int32_t hidden, int32_t n_experts, int32_t top_k, float* __restrict__ logits,
    int32_t* __restrict__ arrivals, void* __restrict__ ids, int ids64, void* __restrict__ weights,
    int wbf16) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + wave;
  const int t0 = blockIdx.y * kTokBlock;
  const int nt = min(kTokBlock, tokens - t0);
  if (e < n_experts) {
    const int nv = hidden >> 3;                 // 16-byte vectors per row
    const uint4* wr = reinterpret_cast<const uint4*>(w + static_cast<int64_t>(e) * hidden);
    double acc[kTokBlock] = {0.0, 0.0, 0.0, 0.0};
    for (int i = lane; i < nv; i += 64) {
      const uint4 b = wr[i];
      const uint32_t bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int tt = 0; tt < kTokBlock; ++tt) {
        if (tt < nt) {
          const uint4 a = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(t0 + tt) * hidden)[i];
          const uint32_t av[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float a0 = __uint_as_float(av[j] << 16), a1 = __uint_as_float(av[j] & 0xffff0000u);
            const float b0 = __uint_as_float(bv[j] << 16), b1 = __uint_as_float(bv[j] & 0xffff0000u);
            acc[tt] += static_cast<double>(a0 * b0);     // exact products
            acc[tt] += static_cast<double>(a1 * b1);
          }
        }
      }
    }
#pragma unroll
    for (int tt = 0; tt < kTokBlock; ++tt) {
      const double s = wave_sum_f64(acc[tt]);
      if (lane == 0 && tt < nt) {
        float l = static_cast<float>(s);
        if (bias) l += bias[e];
        logits[static_cast<int64_t>(t0 + tt) * n_experts + e] = l;
      }
    }
  }
  // the last workgroup of this token block selects
  __shared__ int last;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(&arrivals[blockIdx.y], 1);
    last = prev == static_cast<int>(gridDim.x) - 1;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  if (wave < nt) {
    const int64_t t = t0 + wave;
    topk_one_token<PER>(logits + t * n_experts, n_experts, top_k, t, ids, ids64, weights, wbf16);
  }
  if (threadIdx.x == 0) arrivals[blockIdx.y] = 0;
}

}  // namespace moe

extern "C" int moe_router_topk(const void* x, const void* w, const float* bias, int32_t tokens,
                               int32_t hidden, int32_t n_experts, int32_t top_k, float* logits,
                               int32_t* arrivals, void* ids, int32_t ids_dtype, void* weights,
                               int32_t w_dtype, void* stream) {
  MOE_REQUIRE(x && w && logits && arrivals && ids && weights, "moe_router_topk: NULL pointer");
  MOE_REQUIRE(tokens >= 0, "moe_router_topk: tokens < 0");
  MOE_REQUIRE(hidden > 0 && hidden % 8 == 0, "moe_router_topk: hidden %% 8 != 0 (%d)", hidden);
  MOE_REQUIRE(top_k >= 1 && top_k <= moe::kMaxTopK && top_k <= n_experts && n_experts <= 4096,
              "moe_router_topk: need 1 <= top_k <= min(32, n_experts), n_experts <= 4096");
  MOE_REQUIRE(ids_dtype == MOE_I32 || ids_dtype == MOE_I64, "moe_router_topk: bad ids_dtype");
  MOE_REQUIRE(w_dtype == MOE_F32 || w_dtype == MOE_BF16, "moe_router_topk: bad w_dtype");
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0,
              "moe_router_topk: x and w must be 16-byte aligned");
  if (tokens == 0) return MOE_OK;
  const dim3 grid((n_experts + 3) / 4, (tokens + moe::kTokBlock - 1) / moe::kTokBlock);
  MOE_REQUIRE(grid.y <= 65535, "moe_router_topk: too many tokens (%d)", tokens);
  hipStream_t s = moe::as_stream(stream);
  const int i64 = ids_dtype == MOE_I64 ? 1 : 0, bf = w_dtype == MOE_BF16 ? 1 : 0;
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* wp = static_cast<const uint16_t*>(w);
  if (n_experts <= 256)
    hipLaunchKernelGGL(moe::router_kernel<4>, grid, dim3(256), 0, s, xp, wp, bias, tokens, hidden,
                       n_experts, top_k, logits, arrivals, ids, i64, weights, bf);
  else if (n_experts <= 1024)
    hipLaunchKernelGGL(moe::router_kernel<16>, grid, dim3(256), 0, s, xp, wp, bias, tokens,
                       hidden, n_experts, top_k, logits, arrivals, ids, i64, weights, bf);
  else
    hipLaunchKernelGGL(moe::router_kernel<64>, grid, dim3(256), 0, s, xp, wp, bias, tokens,
                       hidden, n_experts, top_k, logits, arrivals, ids, i64, weights, bf);
  return moe::check_launch("moe_router_topk");
}
