// Device-resident expert slot table: one layer's LRU, updated on the GPU so
// that no host sync sits inside a captured decode step.
//
// Table (one per layer):
//   slot_of[E]      int32  expert -> slot, -1 absent
//   slot_expert[C]  int32  slot -> expert, -1 empty
//   slot_stamp[C]   int64  step at which the slot was last used
//   step[1]         int64  bumped on the device by every resolve
//
// Decisions are exactly those of bin/devcache.py:65-98: a miss takes the slot
// with the smallest stamp, the lowest index winning a tie.  Slots used in the
// current step hold the largest stamp, so none of them can be evicted by a
// later id of the same call.
//
// One wavefront does the whole resolve.  The ids are processed in order (two
// simultaneous misses must not get the same slot), but nothing in the loop
// waits on memory: stamps and slot owners live in registers (C/64 slots per
// lane), lane r holds id r and its slot as loaded at the start, and every
// eviction or assignment is applied to the later lanes' copies at once, so
// each lane sees exactly the table the sequential reference loop would.  The
// victim search is a wave-wide arg-min instead of a C-element scan.  Lane 0
// issues the table writes in program order.
#include "common.hpp"

namespace moe {

constexpr int kMaxCap = 4096;
constexpr int kPerLane = kMaxCap / 64;

__global__ __launch_bounds__(256) void slots_init_kernel(int32_t* slot_of, int32_t n_experts,
                                                         int32_t* slot_expert, int64_t* stamp,
                                                         int32_t cap, int64_t* step) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n_experts) slot_of[i] = -1;
  if (i < cap) {
    slot_expert[i] = -1;
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
  const int lane = threadIdx.x;
  // Slot c = lane + 64*j lives in lane's registers: its stamp and its expert.
  int64_t st[PER];
  int32_t se[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = lane + 64 * j;
    st[j] = c < cap ? stamp[c] : INT64_MAX;
    se[j] = c < cap ? slot_expert[c] : -1;
  }
  // Read at run time, never a launch argument: a captured step would
  // otherwise stamp the same value on every replay.
  const int64_t step = *step_ptr + 1;
  int32_t nm = 0;
  int64_t hits = 0;
  for (int32_t base = 0; base < k; base += 64) {
    // lane r holds id base+r and its current slot (coherent load: lane 0's
    // table writes of the previous chunk are visible after the fence below)
    int32_t my_e = -1, my_s = -1;
    if (base + lane < k) {
      my_e = ids64 ? static_cast<int32_t>(reinterpret_cast<const int64_t*>(ids)[base + lane])
                   : reinterpret_cast<const int32_t*>(ids)[base + lane];
      if (my_e >= 0 && my_e < n_experts)
        my_s = __hip_atomic_load(slot_of + my_e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        my_e = -1;
    }
    const int n = min(64, k - base);
    for (int r = 0; r < n; ++r) {
      const int32_t e = __shfl(my_e, r, 64);
      int32_t s = __shfl(my_s, r, 64);
      if (e < 0) {                                  // cannot index slot_of: report, skip
        if (lane == 0) out_slot[base + r] = -1;
        continue;
      }
      if (s < 0) {
        // arg-min over (stamp, slot) across the wave: lowest slot wins a tie
        int64_t bst = INT64_MAX;
        int32_t bix = INT32_MAX;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
          const int c = lane + 64 * j;
          if (c < cap && st[j] < bst) { bst = st[j]; bix = c; }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const int64_t ost = __shfl_xor(bst, o, 64);
          const int32_t oix = __shfl_xor(bix, o, 64);
          if (ost < bst || (ost == bst && oix < bix)) { bst = ost; bix = oix; }
        }
        s = bix;
        int32_t vloc = -1;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
          if (j == (s >> 6)) {
            vloc = se[j];
            if ((s & 63) == lane) se[j] = e;
          }
        }
        const int32_t victim = __shfl(vloc, s & 63, 64);
        // later ids of this call see the table as it is now
        if (lane > r) {
          if (my_e == victim) my_s = -1;
          if (my_e == e) my_s = s;
        }
        if (lane == 0) {
          if (victim >= 0) slot_of[victim] = -1;
          slot_of[e] = s;
          slot_expert[s] = e;
          fetch_slot[nm] = s;
          fetch_expert[nm] = e;
        }
        ++nm;
      } else {
        ++hits;
      }
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (j == (s >> 6) && (s & 63) == lane) st[j] = step;
      if (lane == 0) out_slot[base + r] = s;
    }
    __threadfence();
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = lane + 64 * j;
    if (c < cap) stamp[c] = st[j];
  }
  if (lane == 0) {
    *step_ptr = step;
    *nmiss_ptr = nm;
    if (stats) {
      stats[0] += hits;
      stats[1] += nm;
    }
  }
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
  hipStream_t s = moe::as_stream(stream);
  const int ids64 = ids_dtype == MOE_I64;
  if (cap <= 256) {
    hipLaunchKernelGGL(moe::resolve_kernel<4>, dim3(1), dim3(64), 0, s, ids, ids64, k, slot_of,
                       n_experts, slot_expert, slot_stamp, cap, step, out_slot, fetch_slot,
                       fetch_expert, nmiss, stats);
  } else if (cap <= 1024) {
    hipLaunchKernelGGL(moe::resolve_kernel<16>, dim3(1), dim3(64), 0, s, ids, ids64, k, slot_of,
                       n_experts, slot_expert, slot_stamp, cap, step, out_slot, fetch_slot,
                       fetch_expert, nmiss, stats);
  } else {
    hipLaunchKernelGGL(moe::resolve_kernel<moe::kPerLane>, dim3(1), dim3(64), 0, s, ids, ids64,
                       k, slot_of, n_experts, slot_expert, slot_stamp, cap, step, out_slot,
                       fetch_slot, fetch_expert, nmiss, stats);
  }
  return moe::check_launch("moe_resolve_slots");
}

}  // extern "C"
