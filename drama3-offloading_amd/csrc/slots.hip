// Device-resident expert slot table: one layer's LRU, updated on the GPU so
// that no host sync sits inside a captured decode step.
//
// Table (one per layer):
//   slot_of[E]      int32  expert -> slot, -1 absent
//   slot_expert[C]  int32  slot -> expert, -1 empty
//   slot_stamp[C]   int64  step at which the slot was last used
//   step[1]         int64  bumped on the device by every resolve
//
// The resolve itself (one wavefront, decisions identical to
// bin/devcache.py:65-98) is in resolve.hpp.
#include "common.hpp"
#include "resolve.hpp"

namespace moe {

__global__ __launch_bounds__(256) void slots_init_kernel(int32_t* slot_of, int32_t n_experts,
                                                         int32_t* slot_expert, int64_t* stamp,
                                                         int32_t cap, int64_t* step) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n_experts) slot_of[i] = -1;
  if (i < cap) {
    slot_expert[i] = -1;
    // distinct negative stamps: the first `cap` misses take slots 0, 1, 2, ...
    stamp[i] = -static_cast<int64_t>(cap - i);
  }
  if (i == 0) *step = 0;
}

template <int PER>
__global__ __launch_bounds__(64) void resolve_kernel(
    const void* __restrict__ ids, int ids64, int32_t k, int32_t* __restrict__ slot_of,
    int32_t n_experts, int32_t* __restrict__ slot_expert, int64_t* __restrict__ stamp,
    int32_t cap, int64_t* __restrict__ step_ptr, int32_t* __restrict__ out_slot,
    int32_t* __restrict__ fetch_slot, int32_t* __restrict__ fetch_expert,
    int32_t* __restrict__ nmiss_ptr, int64_t* __restrict__ stats) {
  auto id_at = [ids, ids64](int i) -> int32_t {
    return ids64 ? static_cast<int32_t>(reinterpret_cast<const int64_t*>(ids)[i])
                 : reinterpret_cast<const int32_t*>(ids)[i];
  };
  resolve_wave_impl<PER>(id_at, k, n_experts, slot_of, slot_expert, stamp, cap, step_ptr,
                         out_slot, fetch_slot, fetch_expert, nmiss_ptr, stats);
}

}  // namespace moe

extern "C" {

int moe_slots_init(int32_t* slot_of, int32_t n_experts, int32_t* slot_expert,
                   int64_t* slot_stamp, int32_t cap, int64_t* step, void* stream) {
  MOE_REQUIRE(slot_of && slot_expert && slot_stamp && step, "moe_slots_init: NULL pointer");
  MOE_REQUIRE(n_experts >= 1 && cap >= 1 && cap <= moe::kMaxCap,
              "moe_slots_init: need n_experts >= 1 and 1 <= cap <= %d (got %d, %d)",
              moe::kMaxCap, n_experts, cap);
  int n = n_experts > cap ? n_experts : cap;
  hipLaunchKernelGGL(moe::slots_init_kernel, dim3((n + 255) / 256), dim3(256), 0,
                     moe::as_stream(stream), slot_of, n_experts, slot_expert, slot_stamp, cap,
                     step);
  return moe::check_launch("moe_slots_init");
}

int moe_resolve_slots(const void* ids, int32_t ids_dtype, int32_t k, int32_t* slot_of,
                      int32_t n_experts, int32_t* slot_expert, int64_t* slot_stamp, int32_t cap,
                      int64_t* step, int32_t* out_slot, int32_t* fetch_slot,
                      int32_t* fetch_expert, int32_t* nmiss, int64_t* stats, void* stream) {
  MOE_REQUIRE(ids && slot_of && slot_expert && slot_stamp && step && out_slot && fetch_slot &&
                  fetch_expert && nmiss,
              "moe_resolve_slots: NULL pointer");
  MOE_REQUIRE(ids_dtype == MOE_I32 || ids_dtype == MOE_I64,
              "moe_resolve_slots: ids_dtype must be MOE_I32 or MOE_I64");
  MOE_REQUIRE(k >= 0, "moe_resolve_slots: k < 0");
  MOE_REQUIRE(n_experts >= 1 && cap >= 1 && cap <= moe::kMaxCap,
              "moe_resolve_slots: need n_experts >= 1 and 1 <= cap <= %d (got %d, %d)",
              moe::kMaxCap, n_experts, cap);
  // more ids than slots would hand one slot to two ids of this call
  MOE_REQUIRE(k <= cap, "moe_resolve_slots: k (%d) exceeds the cache capacity (%d)", k, cap);
  hipStream_t s = moe::as_stream(stream);
  const int ids64 = ids_dtype == MOE_I64;
#define MOE_RS(PER)                                                                              \
  hipLaunchKernelGGL(moe::resolve_kernel<PER>, dim3(1), dim3(64), 0, s, ids, ids64, k, slot_of,  \
                     n_experts, slot_expert, slot_stamp, cap, step, out_slot, fetch_slot,         \
                     fetch_expert, nmiss, stats)
  if (cap <= 256) MOE_RS(4);
  else if (cap <= 1024) MOE_RS(16);
  else MOE_RS(64);
#undef MOE_RS
  return moe::check_launch("moe_resolve_slots");
}

}  // extern "C"
