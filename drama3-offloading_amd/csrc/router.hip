// Top-k-of-E router: logits = x . W^T (+ bias), top-k by descending logit
// (ties to the lower expert), softmax over the k selected (== softmax over all
// E then renormalise, upstream's norm_topk_prob).
//
// Logit arithmetic: a bf16 x bf16 product is exact in float32; products are
// summed in float64 and rounded once to float32.  With float64 partial sums
// exact for ordinary data, the rounded logit does not depend on the order of
// summation, which is what lets expert ids match the oracle bit for bit.
#include "common.hpp"

namespace moe {

constexpr int kMaxTopK = 32;

// One wave per (token, expert): 16-byte loads of x and W rows, float64 sum.
__global__ __launch_bounds__(256) void router_logits_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const float* __restrict__ bias,
    int32_t tokens, int32_t hidden, int32_t n_experts, float* __restrict__ logits) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + wave;
  const int t = blockIdx.y;
  if (e >= n_experts) return;
  const uint4* xr = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(t) * hidden);
  const uint4* wr = reinterpret_cast<const uint4*>(w + static_cast<int64_t>(e) * hidden);
  const int nv = hidden >> 3;
  double acc = 0.0;
  for (int i = lane; i < nv; i += 64) {
    uint4 a = xr[i];
    uint4 b = wr[i];
    const uint32_t av[4] = {a.x, a.y, a.z, a.w};
    const uint32_t bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float a0 = __uint_as_float(av[j] << 16), a1 = __uint_as_float(av[j] & 0xffff0000u);
      float b0 = __uint_as_float(bv[j] << 16), b1 = __uint_as_float(bv[j] & 0xffff0000u);
      acc += static_cast<double>(a0 * b0);   // exact products
      acc += static_cast<double>(a1 * b1);
    }
  }
  acc = wave_sum_f64(acc);
  if (lane == 0) {
    float l = static_cast<float>(acc);
    if (bias) l += bias[e];
    logits[static_cast<int64_t>(t) * n_experts + e] = l;
  }
}

// One wave per token: k rounds of wave arg-max over the logits in LDS.
__global__ __launch_bounds__(64) void router_topk_kernel(const float* __restrict__ logits,
                                                         int32_t n_experts, int32_t top_k,
                                                         void* __restrict__ ids, int ids64,
                                                         void* __restrict__ weights, int wbf16) {
  extern __shared__ unsigned char smem[];
  float* lg = reinterpret_cast<float*>(smem);
  unsigned char* taken = smem + sizeof(float) * n_experts;
  const int lane = threadIdx.x;
  const int t = blockIdx.x;
  const float* row = logits + static_cast<int64_t>(t) * n_experts;
  for (int e = lane; e < n_experts; e += 64) {
    lg[e] = row[e];
    taken[e] = 0;
  }
  __syncthreads();
  float sel_v[kMaxTopK];
  int sel_i[kMaxTopK];
  for (int r = 0; r < top_k; ++r) {
    float bv = -INFINITY;
    int bi = INT32_MAX;
    for (int e = lane; e < n_experts; e += 64) {
      if (taken[e]) continue;
      float v = lg[e];
      if (bi == INT32_MAX || v > bv || (v == bv && e < bi)) { bv = v; bi = e; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      float ov = __shfl_xor(bv, o, 64);
      int oi = __shfl_xor(bi, o, 64);
      bool better = (oi != INT32_MAX) && (bi == INT32_MAX || ov > bv || (ov == bv && oi < bi));
      if (better) { bv = ov; bi = oi; }
    }
    if (lane == 0 && bi != INT32_MAX) taken[bi] = 1;
    __syncthreads();
    sel_v[r] = bv;
    sel_i[r] = bi;
  }
  if (lane == 0) {
    const float m = sel_v[0];
    float ex[kMaxTopK];
    float sum = 0.0f;
    for (int r = 0; r < top_k; ++r) {
      ex[r] = expf(sel_v[r] - m);
      sum += ex[r];
    }
    for (int r = 0; r < top_k; ++r) {
      const int64_t o = static_cast<int64_t>(t) * top_k + r;
      if (ids64) reinterpret_cast<int64_t*>(ids)[o] = sel_i[r];
      else reinterpret_cast<int32_t*>(ids)[o] = sel_i[r];
      const float wv = ex[r] / sum;
      if (wbf16) reinterpret_cast<uint16_t*>(weights)[o] = f32_to_bf16(wv);
      else reinterpret_cast<float*>(weights)[o] = wv;
    }
  }
}

}  // namespace moe

extern "C" int moe_router_topk(const void* x, const void* w, const float* bias, int32_t tokens,
                               int32_t hidden, int32_t n_experts, int32_t top_k, float* logits,
                               void* ids, int32_t ids_dtype, void* weights, int32_t w_dtype,
                               void* stream) {
  MOE_REQUIRE(x && w && logits && ids && weights, "moe_router_topk: NULL pointer");
  MOE_REQUIRE(tokens >= 0, "moe_router_topk: tokens < 0");
  MOE_REQUIRE(hidden > 0 && hidden % 8 == 0, "moe_router_topk: hidden %% 8 != 0 (%d)", hidden);
  MOE_REQUIRE(top_k >= 1 && top_k <= moe::kMaxTopK && top_k <= n_experts && n_experts <= 4096,
              "moe_router_topk: need 1 <= top_k <= min(32, n_experts), n_experts <= 4096");
  MOE_REQUIRE(ids_dtype == MOE_I32 || ids_dtype == MOE_I64, "moe_router_topk: bad ids_dtype");
  MOE_REQUIRE(w_dtype == MOE_F32 || w_dtype == MOE_BF16, "moe_router_topk: bad w_dtype");
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0,
              "moe_router_topk: x and w must be 16-byte aligned");
  if (tokens == 0) return MOE_OK;
  hipStream_t s = moe::as_stream(stream);
  hipLaunchKernelGGL(moe::router_logits_kernel, dim3((n_experts + 3) / 4, tokens), dim3(256), 0, s,
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), bias,
                     tokens, hidden, n_experts, logits);
  int rc = moe::check_launch("moe_router_topk(logits)");
  if (rc) return rc;
  const size_t shm = static_cast<size_t>(n_experts) * (sizeof(float) + 1);
  hipLaunchKernelGGL(moe::router_topk_kernel, dim3(tokens), dim3(64), shm, s, logits, n_experts,
                     top_k, ids, ids_dtype == MOE_I64 ? 1 : 0, weights,
                     w_dtype == MOE_BF16 ? 1 : 0);
  return moe::check_launch("moe_router_topk(topk)");
}
