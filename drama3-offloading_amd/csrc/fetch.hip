// Zero-copy expert fetch: page-locked host records -> HBM cache slots.
//
// Why a kernel and not hipMemcpyAsync: a captured memcpy node bakes its
// source address, so a replayed graph would copy the capture-time experts
// forever (measured as FROZEN in the reference, notes/06-cuda-graphs-plan.md
// :182).  This kernel reads which expert goes to which slot, and how many
// jobs there are, from device memory when it runs.
//
// Shape: grid (blocks_per_job, max_jobs), 256 threads.  Job j = blockIdx.y
// copies expert fetch_expert[j] into slot fetch_slot[j] for every buffer
// pair; jobs with j >= *nmiss retire at once, so the grid can be sized for
// the worst case (every id a miss) and stay static under capture.
//
// Transfer: 16-byte loads per lane, wave-contiguous (a wave instruction
// covers 1 KiB of one record), UNROLL loads in flight per lane before the
// matching stores, so each wave keeps UNROLL KiB of host reads outstanding.
// Pairs whose sizes or addresses are not 16-byte aligned (tiny scale blocks
// of toy shapes) take a 4-byte path in the same launch.
#include "common.hpp"

namespace moe {

constexpr int kFetchThreads = 256;
constexpr int kFetchUnroll = 4;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct FetchArgs {
  const char* src[4];
  char* dst[4];
  int64_t bytes[4];
  int32_t vec16[4];   // 1 if the pair takes the 16-byte path
  int32_t npairs;
};

__global__ __launch_bounds__(kFetchThreads) void fetch_kernel(FetchArgs a,
                                                              const int32_t* __restrict__ fexp,
                                                              const int32_t* __restrict__ fslot,
                                                              const int32_t* __restrict__ nmiss) {
  const int j = blockIdx.y;
  if (j >= *nmiss) return;
  const int64_t e = fexp[j];
  const int64_t s = fslot[j];
  // block b of a job owns the rows b, b + gridDim.x, ... of blockDim.x*UNROLL vectors
  for (int p = 0; p < a.npairs; ++p) {
    const int64_t bytes = a.bytes[p];
    const char* src = a.src[p] + e * bytes;
    char* dst = a.dst[p] + s * bytes;
    if (a.vec16[p]) {
      const int64_t n = bytes >> 4;
      const u32x4* sv = reinterpret_cast<const u32x4*>(src);
      u32x4* dv = reinterpret_cast<u32x4*>(dst);
      const int64_t row = static_cast<int64_t>(blockDim.x) * kFetchUnroll;
      // rows of blockDim*UNROLL vectors are interleaved across the job's blocks
      for (int64_t r0 = blockIdx.x * row; r0 < n; r0 += gridDim.x * row) {
        const int64_t base = r0 + threadIdx.x;
        if (r0 + row <= n) {
          u32x4 v[kFetchUnroll];
#pragma unroll
          for (int u = 0; u < kFetchUnroll; ++u)
            v[u] = __builtin_nontemporal_load(sv + base + u * blockDim.x);
#pragma unroll
          for (int u = 0; u < kFetchUnroll; ++u) dv[base + u * blockDim.x] = v[u];
        } else {
          for (int64_t i = base; i < n && i < r0 + row; i += blockDim.x) dv[i] = sv[i];
        }
      }
    } else {
      const int64_t n = bytes >> 2;
      const uint32_t* sw = reinterpret_cast<const uint32_t*>(src);
      uint32_t* dw = reinterpret_cast<uint32_t*>(dst);
      for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
           i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        dw[i] = sw[i];
    }
  }
}

}  // namespace moe

extern "C" int moe_fetch(const moe_fetch_pair* pairs, int32_t npairs,
                         const int32_t* fetch_expert, const int32_t* fetch_slot,
                         const int32_t* nmiss, int32_t max_jobs, int32_t blocks_per_job,
                         void* stream) {
  MOE_REQUIRE(pairs != nullptr, "moe_fetch: pairs is NULL");
  MOE_REQUIRE(npairs >= 1 && npairs <= 4, "moe_fetch: need 1 <= npairs <= 4 (got %d)", npairs);
  MOE_REQUIRE(fetch_expert && fetch_slot && nmiss, "moe_fetch: NULL job list");
  MOE_REQUIRE(max_jobs >= 1 && max_jobs <= 65535, "moe_fetch: need 1 <= max_jobs <= 65535");
  MOE_REQUIRE(blocks_per_job >= 1 && blocks_per_job <= 65535,
              "moe_fetch: need 1 <= blocks_per_job <= 65535");
  moe::FetchArgs a = {};
  a.npairs = npairs;
  for (int p = 0; p < npairs; ++p) {
    const uintptr_t sa = reinterpret_cast<uintptr_t>(pairs[p].src);
    const uintptr_t da = reinterpret_cast<uintptr_t>(pairs[p].dst);
    const int64_t b = pairs[p].bytes;
    MOE_REQUIRE(pairs[p].src && pairs[p].dst, "moe_fetch: pair %d has a NULL buffer", p);
    MOE_REQUIRE(b > 0, "moe_fetch: pair %d has %lld bytes per record", p, (long long)b);
    MOE_REQUIRE(b % 4 == 0 && sa % 4 == 0 && da % 4 == 0,
                "moe_fetch: pair %d must be 4-byte aligned (bytes %lld, src %p, dst %p)", p,
                (long long)b, pairs[p].src, pairs[p].dst);
    a.src[p] = static_cast<const char*>(pairs[p].src);
    a.dst[p] = static_cast<char*>(pairs[p].dst);
    a.bytes[p] = b;
    a.vec16[p] = (b % 16 == 0 && sa % 16 == 0 && da % 16 == 0) ? 1 : 0;
  }
  hipLaunchKernelGGL(moe::fetch_kernel, dim3(blocks_per_job, max_jobs), dim3(moe::kFetchThreads),
                     0, moe::as_stream(stream), a, fetch_expert, fetch_slot, nmiss);
  return moe::check_launch("moe_fetch");
}
