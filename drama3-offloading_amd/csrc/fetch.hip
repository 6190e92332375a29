// Zero-copy expert fetch: page-locked host records -> HBM cache slots.
//
// Why a kernel and not hipMemcpyAsync: a captured memcpy node bakes its
// source address, so a replayed graph would copy the capture-time experts
// forever (measured as FROZEN in the reference, notes/06-cuda-graphs-plan.md
// :182, and on MI355X by the same A/C/B protocol: a captured copy_ per miss
// from a page-locked pool replays the capture-time experts, this kernel the
// experts set after the capture).  This kernel reads which expert goes to
// which slot, and how many jobs there are, from device memory when it runs.
//
// Work distribution: the nmiss queued records (read at run time) are cut
// into pieces of kFetchThreads * kFetchUnroll 16-byte vectors (8 KiB) per
// buffer pair, and the pieces are dealt round-robin to every workgroup of the
// grid, whatever the miss count.  The grid is deliberately small:
// blocks_per_job * min(max_jobs, 8) workgroups of 128 threads keep about
// 192 KiB of host reads in flight at the default of 3, about the host link's
// bandwidth-delay product (~57 GB/s x ~2-3 us).  Measured on MI355X (Drama-3
// records, 1 / 3 / 8 misses): 53.6 / 56.1 / 56.8 GB/s at 3 workgroups per
// job, 53.6 / 55.8 / 56.4 at 2, 53.1 / 55.9 / 56.8 at 4, 50.9 / 53.4 / 54.0
// at 6, and 51 GB/s with 64 x 256-thread workgroups at 8; the copy engine's
// H2D rate on the same pool is 57.2 GB/s.
//
// Each lane issues kFetchUnroll 16-byte loads, wave-contiguous (one wave
// instruction covers 1 KiB of one record), before the matching stores.
// Pairs whose sizes or addresses are not 16-byte aligned (tiny scale blocks
// of toy shapes) are copied in 4-byte words by whole workgroups.
//
// A pair with tile_k = K > 0 holds row-major [rows, K] e4m3 matrices on the
// host and writes them in MFMA tile order: the unit (16 bytes) of row
// 16g + r, column unit c goes to unit
//   ((g * K/128 + c/8) * 2 + c % 2) * 64 + ((c / 2) % 4) * 16 + r
// of the record, which is byte (g*K/128 + b)*2048 + h*1024 + (16q + r)*16 of
// the tile layout (b = c/8, q = (c/2) % 4, h = c % 2).  A piece of such a
// pair is 16 rows x W column units (W = 32, 16 or 8, dividing K/16), whose
// units fill one contiguous run of 16W units of the cache: the piece is read
// as 16 row runs of 16W bytes, transposed through LDS (rows padded by one
// unit, so the 16 rows a wave reads fall in distinct banks) and stored
// contiguously.  Storing the units straight to their scattered places
// writes 64 distinct 128-byte lines per wave instruction and measured 6 %
// below the byte copy's rate.
#include "fetch.hpp"

namespace moe {

__global__ __launch_bounds__(kFetchThreads) void fetch_kernel(FetchArgs a,
                                                              const int32_t* __restrict__ fexp,
                                                              const int32_t* __restrict__ fslot,
                                                              const int32_t* __restrict__ nmiss,
                                                              int32_t max_jobs) {
  __shared__ u32x4 stage[16 * 33];   // one tile-order piece, rows padded by one unit
  // The job of this workgroup's first item is read with the miss count, not
  // after it (the lists hold max_jobs entries), so the count and the first
  // record's expert and slot arrive in one memory round trip.  The values
  // are used only if that item exists.
  const int32_t j_first = min(static_cast<int32_t>(blockIdx.x / static_cast<uint32_t>(a.pieces_per_job)),
                              a.last_job);
  const int32_t e_first = fexp[j_first];
  const int32_t s_first = fslot[j_first];
  int32_t n_raw = *nmiss;
  // the count passes through this (empty) statement with the list values as
  // inputs, so all three loads are issued before anything waits on one: the
  // compiler would otherwise sink the list loads below the no-work branch,
  // or issue one of them after waiting for the count, a second round trip
  asm volatile("" : "+s"(n_raw) : "s"(e_first), "s"(s_first));
  const int32_t nm = min(n_raw, max_jobs);
  const int64_t total = static_cast<int64_t>(nm) * a.pieces_per_job;
  for (int64_t item = blockIdx.x; item < total; item += gridDim.x) {
    const int64_t j = item / a.pieces_per_job;
    const int64_t e = j == j_first ? e_first : fexp[j];
    const int64_t s = j == j_first ? s_first : fslot[j];
    fetch_piece(a, item - j * a.pieces_per_job, e, s, stage);
  }
}

int fetch_args(const moe_fetch_pair* pairs, int32_t npairs, int32_t max_jobs, FetchArgs* out) {
  MOE_REQUIRE(pairs != nullptr, "moe_fetch: pairs is NULL");
  MOE_REQUIRE(npairs >= 1 && npairs <= 4, "moe_fetch: need 1 <= npairs <= 4 (got %d)", npairs);
  FetchArgs a = {};
  a.npairs = npairs;
  a.last_job = max_jobs - 1;
  const int64_t row = static_cast<int64_t>(kFetchThreads) * kFetchUnroll;
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
    const int64_t tk = pairs[p].tile_k;
    MOE_REQUIRE(tk >= 0, "moe_fetch: pair %d has tile_k %lld", p, (long long)tk);
    if (tk > 0) {
      MOE_REQUIRE(tk % 128 == 0 && b % (16 * tk) == 0,
                  "moe_fetch: pair %d: tile_k %lld must be a multiple of 128 and the record "
                  "(%lld bytes) whole groups of 16 rows of it", p, (long long)tk, (long long)b);
      MOE_REQUIRE(a.vec16[p] && (b >> 4) < (1LL << 32),
                  "moe_fetch: pair %d in tile order must be 16-byte aligned with records "
                  "under 64 GiB", p);
    }
    const uint32_t upr = static_cast<uint32_t>(tk / 16);
    a.tile_upr[p] = upr;
    a.tile_wlog[p] = upr % 32 == 0 ? 5 : upr % 16 == 0 ? 4 : 3;
    if (tk > 0)
      a.pieces[p] = (b / tk / 16) * (upr >> a.tile_wlog[p]);
    else
      a.pieces[p] = a.vec16[p] ? ((b >> 4) + row - 1) / row : 1;
    a.pieces_per_job += a.pieces[p];
  }
  *out = a;
  return MOE_OK;
}

}  // namespace moe

extern "C" int moe_fetch(const moe_fetch_pair* pairs, int32_t npairs,
                         const int32_t* fetch_expert, const int32_t* fetch_slot,
                         const int32_t* nmiss, int32_t max_jobs, int32_t blocks_per_job,
                         void* stream) {
  MOE_REQUIRE(fetch_expert && fetch_slot && nmiss, "moe_fetch: NULL job list");
  MOE_REQUIRE(max_jobs >= 1 && max_jobs <= 65535, "moe_fetch: need 1 <= max_jobs <= 65535");
  MOE_REQUIRE(blocks_per_job >= 1 && blocks_per_job <= 4096,
              "moe_fetch: need 1 <= blocks_per_job <= 4096");
  moe::FetchArgs a;
  const int rc = moe::fetch_args(pairs, npairs, max_jobs, &a);
  if (rc != MOE_OK) return rc;
  const int grid = blocks_per_job * (max_jobs < moe::kFetchMaxJobsInGrid ? max_jobs
                                                                          : moe::kFetchMaxJobsInGrid);
  hipLaunchKernelGGL(moe::fetch_kernel, dim3(grid), dim3(moe::kFetchThreads), 0,
                     moe::as_stream(stream), a, fetch_expert, fetch_slot, nmiss, max_jobs);
  return moe::check_launch("moe_fetch");
}
