// Token -> expert grouping (permute), its inverse (unpermute), and the
// torch.unique-style renumbering the reference uses for its gathered subsets.
//
// permute: one workgroup of 1024 threads.  Expert ids are staged through LDS
// as uint16 in chunks; thread i owns experts i, i+1024, ... and scans every
// chunk (all threads read the same LDS word, a broadcast), first counting its
// experts, then -- after a block-wide exclusive scan of the counts -- writing
// the positions of its experts' pairs in pair order.  The order is therefore
// stable by construction and identical on every run, and no atomics or
// cleared counters are needed (graph-safe: nothing to memset).
#include "common.hpp"

namespace moe {

constexpr int kPermThreads = 1024;
constexpr int kPermChunk = 8192;   // ids staged per LDS pass
constexpr int kPermMaxExperts = 4096;
constexpr int kPermPer = kPermMaxExperts / kPermThreads;

__device__ __forceinline__ int32_t read_id(const void* ids, int ids64, int64_t p) {
  return ids64 ? static_cast<int32_t>(reinterpret_cast<const int64_t*>(ids)[p])
               : reinterpret_cast<const int32_t*>(ids)[p];
}

// Exclusive scan over kPermThreads values, returns the total.
__device__ int32_t block_exclusive_scan(int32_t v, int32_t* scratch, int32_t* out_prefix) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int32_t incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int32_t n = __shfl_up(incl, o, 64);
    if (lane >= o) incl += n;
  }
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  if (tid < 16) {
    int32_t w = scratch[tid];
    int32_t wi = w;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      int32_t n = __shfl_up(wi, o, 64);
      if (tid >= o) wi += n;
    }
    scratch[16 + tid] = wi - w;    // exclusive wave offsets
    if (tid == 15) scratch[32] = wi;
  }
  __syncthreads();
  *out_prefix = scratch[16 + wave] + incl - v;
  int32_t total = scratch[32];
  __syncthreads();
  return total;
}

__global__ __launch_bounds__(kPermThreads) void permute_kernel(
    const void* __restrict__ ids, int ids64, int64_t P, int32_t n_experts,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ sorted_pairs,
    int32_t* __restrict__ pair_pos) {
  __shared__ uint16_t sid[kPermChunk];
  __shared__ int32_t scratch[40];
  const int tid = threadIdx.x;
  int32_t cnt[kPermPer];
#pragma unroll
  for (int i = 0; i < kPermPer; ++i) cnt[i] = 0;

  // pass 1: count
  for (int64_t c0 = 0; c0 < P; c0 += kPermChunk) {
    const int n = static_cast<int>(min<int64_t>(kPermChunk, P - c0));
    for (int i = tid; i < n; i += kPermThreads) {
      int32_t e = read_id(ids, ids64, c0 + i);
      sid[i] = (e >= 0 && e < n_experts) ? static_cast<uint16_t>(e) : 0xffff;
    }
    __syncthreads();
    for (int i = 0; i < n; ++i) {
      const int e = sid[i];
#pragma unroll
      for (int j = 0; j < kPermPer; ++j) cnt[j] += (e == tid + j * kPermThreads);
    }
    __syncthreads();
  }
  // exclusive scan over experts in index order: expert x = tid + j*1024
  int32_t base = 0;
  int32_t run[kPermPer];
#pragma unroll
  for (int j = 0; j < kPermPer; ++j) {
    int32_t pre;
    int32_t tot = block_exclusive_scan(cnt[j], scratch, &pre);
    run[j] = base + pre;
    const int x = tid + j * kPermThreads;
    if (x < n_experts) {
      counts[x] = cnt[j];
      offsets[x] = run[j];
    }
    base += tot;
  }
  if (tid == 0) offsets[n_experts] = base;

  // pass 2: place, in pair order
  for (int64_t c0 = 0; c0 < P; c0 += kPermChunk) {
    const int n = static_cast<int>(min<int64_t>(kPermChunk, P - c0));
    for (int i = tid; i < n; i += kPermThreads) {
      int32_t e = read_id(ids, ids64, c0 + i);
      sid[i] = (e >= 0 && e < n_experts) ? static_cast<uint16_t>(e) : 0xffff;
    }
    __syncthreads();
    for (int i = 0; i < n; ++i) {
      const int e = sid[i];
#pragma unroll
      for (int j = 0; j < kPermPer; ++j) {
        if (e == tid + j * kPermThreads) {
          const int32_t pos = run[j]++;
          sorted_pairs[pos] = static_cast<int32_t>(c0 + i);
          pair_pos[c0 + i] = pos;
        }
      }
    }
    __syncthreads();
  }
  // pairs with an out-of-range id have no position
  for (int64_t c0 = 0; c0 < P; c0 += kPermThreads) {
    const int64_t p = c0 + tid;
    if (p < P) {
      int32_t e = read_id(ids, ids64, p);
      if (e < 0 || e >= n_experts) pair_pos[p] = -1;
    }
  }
}

__global__ __launch_bounds__(kPermThreads) void unique_inverse_kernel(
    const void* __restrict__ ids, int ids64, int64_t P, int32_t n_experts,
    const int32_t* __restrict__ counts, int32_t* __restrict__ n_unique, int32_t* __restrict__ uniq,
    int32_t* __restrict__ rank_of, int32_t* __restrict__ inverse) {
  __shared__ int32_t scratch[40];
  __shared__ int32_t srank[kPermMaxExperts];
  const int tid = threadIdx.x;
  int32_t base = 0;
#pragma unroll
  for (int j = 0; j < kPermPer; ++j) {
    const int x = tid + j * kPermThreads;
    const int32_t present = (x < n_experts && counts[x] > 0) ? 1 : 0;
    int32_t pre;
    int32_t tot = block_exclusive_scan(present, scratch, &pre);
    if (x < n_experts) {
      const int32_t r = present ? base + pre : -1;
      srank[x] = r;
      rank_of[x] = r;
      if (present) uniq[base + pre] = x;
    }
    base += tot;
  }
  if (tid == 0) *n_unique = base;
  __syncthreads();
  for (int64_t p = tid; p < P; p += kPermThreads) {
    int32_t e = read_id(ids, ids64, p);
    inverse[p] = (e >= 0 && e < n_experts) ? srank[e] : -1;
  }
}

// out[t][c] = sum_k w[t][k] * y[pair_pos[t*K+k]][c], k in order, float32 -> bf16
__global__ __launch_bounds__(256) void unpermute_kernel(const float* __restrict__ y,
                                                        const int32_t* __restrict__ pair_pos,
                                                        const void* __restrict__ weights,
                                                        int wbf16, int32_t top_k, int32_t hidden,
                                                        uint16_t* __restrict__ out) {
  const int64_t t = blockIdx.y;
  const int c = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (c >= hidden) return;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k = 0; k < top_k; ++k) {
    const int64_t p = t * top_k + k;
    const float w = wbf16 ? bf16_to_f32(reinterpret_cast<const uint16_t*>(weights)[p])
                          : reinterpret_cast<const float*>(weights)[p];
    const int32_t pos = pair_pos[p];
    if (pos < 0) {
      acc = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
      continue;
    }
    const float4 v = *reinterpret_cast<const float4*>(y + static_cast<int64_t>(pos) * hidden + c);
    acc.x += w * v.x;
    acc.y += w * v.y;
    acc.z += w * v.z;
    acc.w += w * v.w;
  }
  uint16_t* o = out + t * hidden + c;
  o[0] = f32_to_bf16(acc.x);
  o[1] = f32_to_bf16(acc.y);
  o[2] = f32_to_bf16(acc.z);
  o[3] = f32_to_bf16(acc.w);
}

}  // namespace moe

using namespace moe;

extern "C" int moe_permute(const void* ids, int32_t ids_dtype, int32_t tokens, int32_t top_k,
                           int32_t n_experts, int32_t* counts, int32_t* offsets,
                           int32_t* sorted_pairs, int32_t* pair_pos, void* stream) {
  MOE_REQUIRE(ids && counts && offsets && sorted_pairs && pair_pos, "moe_permute: NULL pointer");
  MOE_REQUIRE(ids_dtype == MOE_I32 || ids_dtype == MOE_I64, "moe_permute: bad ids_dtype");
  MOE_REQUIRE(tokens >= 0 && top_k >= 1, "moe_permute: need tokens >= 0, top_k >= 1");
  MOE_REQUIRE(n_experts >= 1 && n_experts <= kPermMaxExperts,
              "moe_permute: need 1 <= n_experts <= %d", kPermMaxExperts);
  const int64_t P = static_cast<int64_t>(tokens) * top_k;
  MOE_REQUIRE(P <= (1LL << 24), "moe_permute: too many pairs (%lld)", (long long)P);
  hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(kPermThreads), 0, as_stream(stream), ids,
                     ids_dtype == MOE_I64 ? 1 : 0, P, n_experts, counts, offsets, sorted_pairs,
                     pair_pos);
  return check_launch("moe_permute");
}

extern "C" int moe_unique_inverse(const void* ids, int32_t ids_dtype, int32_t tokens,
                                  int32_t top_k, int32_t n_experts, const int32_t* counts,
                                  int32_t* n_unique, int32_t* uniq, int32_t* rank_of,
                                  int32_t* inverse, void* stream) {
  MOE_REQUIRE(ids && counts && n_unique && uniq && rank_of && inverse,
              "moe_unique_inverse: NULL pointer");
  MOE_REQUIRE(ids_dtype == MOE_I32 || ids_dtype == MOE_I64, "moe_unique_inverse: bad ids_dtype");
  MOE_REQUIRE(tokens >= 0 && top_k >= 1, "moe_unique_inverse: need tokens >= 0, top_k >= 1");
  MOE_REQUIRE(n_experts >= 1 && n_experts <= kPermMaxExperts,
              "moe_unique_inverse: need 1 <= n_experts <= %d", kPermMaxExperts);
  const int64_t P = static_cast<int64_t>(tokens) * top_k;
  hipLaunchKernelGGL(unique_inverse_kernel, dim3(1), dim3(kPermThreads), 0, as_stream(stream), ids,
                     ids_dtype == MOE_I64 ? 1 : 0, P, n_experts, counts, n_unique, uniq, rank_of,
                     inverse);
  return check_launch("moe_unique_inverse");
}

extern "C" int moe_unpermute(const float* y, const int32_t* pair_pos, const void* weights,
                             int32_t w_dtype, int32_t tokens, int32_t top_k, int32_t hidden,
                             void* out, void* stream) {
  MOE_REQUIRE(y && pair_pos && weights && out, "moe_unpermute: NULL pointer");
  MOE_REQUIRE(w_dtype == MOE_F32 || w_dtype == MOE_BF16, "moe_unpermute: bad w_dtype");
  MOE_REQUIRE(tokens >= 0 && top_k >= 1, "moe_unpermute: need tokens >= 0, top_k >= 1");
  MOE_REQUIRE(hidden > 0 && hidden % 4 == 0, "moe_unpermute: hidden %% 4 != 0");
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(y) % 16 == 0, "moe_unpermute: y must be 16-byte aligned");
  if (tokens == 0) return MOE_OK;
  hipLaunchKernelGGL(unpermute_kernel, dim3((hidden / 4 + 255) / 256, tokens), dim3(256), 0,
                     as_stream(stream), y, pair_pos, weights, w_dtype == MOE_BF16 ? 1 : 0, top_k,
                     hidden, static_cast<uint16_t*>(out));
  return check_launch("moe_unpermute");
}
