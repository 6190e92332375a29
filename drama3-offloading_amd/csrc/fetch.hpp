// The expert fetch's pieces: host page-locked records -> HBM cache slots
// (fetch.hip's kernel and the decode step's route + fetch kernel in
// router.hip share them).  The work distribution, the tile-order stores and
// their measurements are described in fetch.hip.
#pragma once

#include "common.hpp"

namespace moe {


constexpr int kFetchThreads = 128;
constexpr int kFetchUnroll = 4;
constexpr int kFetchMaxJobsInGrid = 8;

struct FetchArgs {
  const char* src[4];
  char* dst[4];
  int64_t bytes[4];
  int64_t pieces[4];      // pieces of this pair per record
  int32_t vec16[4];       // 1 if the pair takes the 16-byte path
  uint32_t tile_upr[4];   // tile order: 16-byte units per row (K / 16), 0 for a byte copy
  uint32_t tile_wlog[4];  // tile order: log2 of the column units per piece (5, 4 or 3)
  int32_t npairs;
  int64_t pieces_per_job; // sum of pieces over pairs (< 2^32)
  int32_t last_job;       // max_jobs - 1, beside pieces_per_job (one kernel-argument load)
};

// Piece k (0 <= k < pieces_per_job) of the job copying record e of every
// pair into slot s.  All threads of the workgroup call it with the same
// arguments; it may use `stage` and synchronise the workgroup.
__device__ __forceinline__ void fetch_piece(const FetchArgs& a, int64_t k, int64_t e, int64_t s,
                                            u32x4* stage) {
  int p = 0;
  while (p + 1 < a.npairs && k >= a.pieces[p]) {
    k -= a.pieces[p];
    ++p;
  }
  // the pair and the piece are the workgroup's: kept scalar, the pair's
  // fields are scalar loads, which no wait on the vector memory counter
  // (the previous piece's stores) holds up
  p = __builtin_amdgcn_readfirstlane(p);
  k = static_cast<int64_t>(static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int32_t>(k))));
  const int64_t row = static_cast<int64_t>(kFetchThreads) * kFetchUnroll;   // vectors per piece
  const int64_t bytes = a.bytes[p];
  const char* src = a.src[p] + e * bytes;
  char* dst = a.dst[p] + s * bytes;
  const uint32_t upr = a.tile_upr[p];
  if (upr != 0) {
    // piece k = (row group g, column units [jW, jW + W)); its destination
    // is the contiguous run of 16W units at unit (g * upr + jW) * 16
    const uint32_t wl = a.tile_wlog[p];
    const uint32_t W = 1u << wl;
    const uint32_t per_g = upr >> wl;
    const uint32_t g = static_cast<uint32_t>(k) / per_g;
    const uint32_t jw = (static_cast<uint32_t>(k) - g * per_g) * W;
    const u32x4* sv = reinterpret_cast<const u32x4*>(src) + (static_cast<int64_t>(g) * 16 * upr + jw);
    u32x4* dv = reinterpret_cast<u32x4*>(dst) + (static_cast<int64_t>(g) * upr + jw) * 16;
    const uint32_t n = 16 * W;   // <= kFetchThreads * kFetchUnroll
    u32x4 v[kFetchUnroll];
    // every lane loads (slots past n repeat the last unit), so the loads
    // issue back to back and no branch splits them
#pragma unroll
    for (int u = 0; u < kFetchUnroll; ++u) {
      const uint32_t i = min(threadIdx.x + u * kFetchThreads, n - 1);
      v[u] = __builtin_nontemporal_load(sv + (i >> wl) * upr + (i & (W - 1)));
    }
#pragma unroll
    for (int u = 0; u < kFetchUnroll; ++u) {
      const uint32_t i = threadIdx.x + u * kFetchThreads;
      if (i < n) stage[(i >> wl) * (W + 1) + (i & (W - 1))] = v[u];
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kFetchUnroll; ++u) {
      // destination unit d = (2 * bb + h) * 64 + 16q + r holds row r, column unit 8bb + 2q + h
      const uint32_t d = threadIdx.x + u * kFetchThreads;
      if (d < n) {
        const uint32_t bh = d >> 6, q = (d >> 4) & 3, r = d & 15;
        dv[d] = stage[r * (W + 1) + (bh >> 1) * 8 + 2 * q + (bh & 1)];
      }
    }
    __syncthreads();
  } else if (a.vec16[p]) {
    const int64_t n = bytes >> 4;
    const u32x4* sv = reinterpret_cast<const u32x4*>(src);
    u32x4* dv = reinterpret_cast<u32x4*>(dst);
    const int64_t r0 = k * row;
    const int64_t base = r0 + threadIdx.x;
    if (r0 + row <= n) {
      u32x4 v[kFetchUnroll];
#pragma unroll
      for (int u = 0; u < kFetchUnroll; ++u)
        v[u] = __builtin_nontemporal_load(sv + base + u * kFetchThreads);
#pragma unroll
      for (int u = 0; u < kFetchUnroll; ++u) dv[base + u * kFetchThreads] = v[u];
    } else {
      for (int64_t i = base; i < n; i += kFetchThreads) dv[i] = sv[i];
    }
  } else {
    const int64_t n = bytes >> 2;
    const uint32_t* sw = reinterpret_cast<const uint32_t*>(src);
    uint32_t* dw = reinterpret_cast<uint32_t*>(dst);
    for (int64_t i = threadIdx.x; i < n; i += kFetchThreads) dw[i] = sw[i];
  }
}

// FetchArgs of a call from its pairs (the checks of moe_fetch).  Returns
// MOE_OK, or MOE_EINVAL with the reason in moe_last_error().
int fetch_args(const moe_fetch_pair* pairs, int32_t npairs, int32_t max_jobs, FetchArgs* out);

}  // namespace moe
