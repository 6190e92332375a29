// The slot-table resolve of one call, by one wavefront (shared by the
// standalone resolve kernel and the fused top-k + resolve decode kernel).
//
// Decisions are exactly those of bin/devcache.py:65-98: step += 1; each id
// in order: a hit stamps its slot; a miss takes the slot with the smallest
// stamp (the lowest index on a tie), evicts that slot's expert and queues
// (slot, expert) for the fetch.  Slots used in the current step carry the
// largest stamp, so no later id of the same call can take them.
//
// Nothing in the loop waits on memory: slot stamps and owners live in
// registers (C/64 slots per lane), lane r holds id r of the current chunk of
// 64 and its slot as it was at the start of the chunk, and every eviction or
// assignment is applied to the later lanes' copies immediately, so each id
// sees exactly the table the sequential loop would.  The victim search is a
// wave-wide arg-min.  Lane 0 issues the table writes, in program order.
#pragma once

#include "common.hpp"

namespace moe {

constexpr int kMaxCap = 4096;

// Slot stamps and owners of a table, slot c = lane + 64*j in lane's register j.
template <int PER>
struct SlotRegs {
  int64_t st[PER];
  int32_t se[PER];

  // Every lane loads (slots past cap read the last one again and drop it):
  // no load under a branch, so all of them are in flight together.
  __device__ __forceinline__ void load(const int64_t* stamp, const int32_t* slot_expert,
                                       int32_t cap) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int c = min(lane + 64 * j, cap - 1);
      st[j] = stamp[c];
      se[j] = slot_expert[c];
    }
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if (lane + 64 * j >= cap) {
        st[j] = INT64_MAX;
        se[j] = -1;
      }
    }
  }
};

// slot_of of an expert table of at most 64*PER entries, entry x in lane x%64's
// register x/64; lookup(x) for a per-lane x via PER shuffles.
template <int PER>
struct ExpertRegs {
  int32_t so[PER];

  __device__ __forceinline__ void load(const int32_t* slot_of, int32_t n_experts) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < PER; ++j) so[j] = slot_of[min(lane + 64 * j, n_experts - 1)];
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (lane + 64 * j >= n_experts) so[j] = -1;
  }
  // entry x = v (held by lane x % 64)
  __device__ __forceinline__ void set(int32_t x, int32_t v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if ((x >> 6) == j && (x & 63) == lane) so[j] = v;
  }
  __device__ __forceinline__ int32_t lookup(int32_t x) const {
    int32_t r = -1;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int32_t v = __shfl(so[j], x & 63, 64);
      if ((x >> 6) == j) r = v;
    }
    return r;
  }
};

// The miss of id e: the victim slot (smallest stamp, lowest slot on a tie,
// one wave-wide min of (stamp + 4096) << 12 | slot; stamps start at
// -cap >= -4096 and grow by one per call, so they stay far below 2^51) is
// returned with its previous owner (-1 when it was empty); e becomes its
// owner in the registers.
template <int PER>
__device__ __forceinline__ int32_t take_victim(SlotRegs<PER>& t, int32_t e, int32_t cap,
                                               int32_t* victim) {
  const int lane = threadIdx.x & 63;
  uint64_t mine = ~0ull;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = lane + 64 * j;
    const uint64_t k =
        c < cap ? (static_cast<uint64_t>(t.st[j] + kMaxCap) << 12) | static_cast<uint64_t>(c) : ~0ull;
    mine = k < mine ? k : mine;
  }
  const int32_t s = static_cast<int32_t>(wave_reduce_u64<false>(mine) & 0xfffull);
  int32_t vloc = -1;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (j == (s >> 6)) {
      vloc = t.se[j];
      if ((s & 63) == lane) t.se[j] = e;
    }
  }
  *victim = lane_value(vloc, s & 63);
  return s;
}

// Resolve one chunk of <= 64 ids (lane r: my_e = id r, my_s = its slot now).
// Returns nothing; updates the registers, the table in memory (lane 0), the
// outputs, and nm / hits.
template <int PER>
__device__ __forceinline__ void resolve_chunk(SlotRegs<PER>& t, int32_t my_e, int32_t my_s,
                                              int n, int32_t base, int64_t step, int32_t cap,
                                              int32_t* __restrict__ slot_of,
                                              int32_t* __restrict__ slot_expert,
                                              int32_t* __restrict__ out_slot,
                                              int32_t* __restrict__ fetch_slot,
                                              int32_t* __restrict__ fetch_expert, int32_t& nm,
                                              int64_t& hits) {
  const int lane = threadIdx.x & 63;
  for (int r = 0; r < n; ++r) {
    const int32_t e = lane_value(my_e, r);
    int32_t s = lane_value(my_s, r);
    if (e < 0) {
      if (lane == 0) out_slot[base + r] = -1;
      continue;
    }
    if (s < 0) {
      int32_t victim;
      s = take_victim(t, e, cap, &victim);
      if (lane > r) {                      // later ids see the table as it is now
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
      if (j == (s >> 6) && (s & 63) == lane) t.st[j] = step;
    if (lane == 0) out_slot[base + r] = s;
  }
}

// The resolve of one chunk of <= 64 ids on register copies of the whole
// table (slot_of in x, slots in t), for a kernel whose workgroups all make
// the decisions and one of them writes the next table out: the decisions of
// resolve_chunk, nothing written to the table in memory.  Lane r ends with
// id r's slot in slot_r (-1 for an id out of range) and miss_r set when id r
// missed; the misses are appended to job_e / job_s, and their positions r
// to job_k when it is given, by lane 0.
//
// The stamps this call gives are kept as one bit per slot register
// (`touched`) and written into t.st at the end, and a miss's victim comes
// from 32-bit keys, (age << 12) | (4095 - slot) with age = step - stamp (0
// for a slot touched by this call), whose wave maximum is the smallest
// stamp, lowest slot on a tie.  An age outside [0, kAgeMax) is keyed as
// kAgeMax; when such a key wins, the victim is taken from the 64-bit
// stamps instead (take_victim on the stamps as they stand), so the
// decisions are resolve_chunk's for every table.
constexpr uint32_t kAgeMax = (1u << 20) - 1;

template <int PER>
__device__ __forceinline__ int32_t take_victim_age(SlotRegs<PER>& t, const uint32_t (&vkey)[PER],
                                                   uint32_t touched, int32_t e, int32_t cap,
                                                   int64_t step, int32_t* victim) {
  const int lane = threadIdx.x & 63;
  uint32_t mine = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t k = ((touched >> j) & 1u) ? (vkey[j] & 4095u) : vkey[j];
    mine = k > mine ? k : mine;
  }
  const uint32_t m = wave_max_u32(mine);
  if ((m >> 12) != kAgeMax) {
    const int32_t s = 4095 - static_cast<int32_t>(m & 4095u);
    int32_t vloc = -1;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if (j == (s >> 6)) {
        vloc = t.se[j];
        if ((s & 63) == lane) t.se[j] = e;
      }
    }
    *victim = lane_value(vloc, s & 63);
    return s;
  }
  // an age past kAgeMax (or a stamp after the step): the 64-bit stamps,
  // with this call's stamps applied
  SlotRegs<PER> u = t;
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if ((touched >> j) & 1u) u.st[j] = step;
  const int32_t s = take_victim(u, e, cap, victim);
#pragma unroll
  for (int j = 0; j < PER; ++j) t.se[j] = u.se[j];
  return s;
}

template <int PER, int PERC>
__device__ __forceinline__ void resolve_regs(SlotRegs<PERC>& t, ExpertRegs<PER>& x, int32_t my_e,
                                             int32_t my_s, int n, int64_t step, int32_t cap,
                                             int32_t* job_e, int32_t* job_s, int32_t* job_k,
                                             int32_t& nm, int64_t& hits, int32_t& slot_r,
                                             bool& miss_r) {
  const int lane = threadIdx.x & 63;
  slot_r = -1;
  miss_r = false;
  uint32_t vkey[PERC];
#pragma unroll
  for (int j = 0; j < PERC; ++j) {
    const int c = lane + 64 * j;
    const int64_t age = step - t.st[j];
    const uint32_t a = (age >= 0 && age < kAgeMax) ? static_cast<uint32_t>(age) : kAgeMax;
    vkey[j] = c < cap ? (a << 12) | static_cast<uint32_t>(4095 - c) : 0u;
  }
  uint32_t touched = 0;
  for (int r = 0; r < n; ++r) {
    const int32_t e = lane_value(my_e, r);
    int32_t s = lane_value(my_s, r);
    if (e < 0) continue;
    if (s < 0) {
      int32_t victim;
      s = take_victim_age(t, vkey, touched, e, cap, step, &victim);
      if (lane > r) {                      // later ids see the table as it is now
        if (my_e == victim) my_s = -1;
        if (my_e == e) my_s = s;
      }
      if (victim >= 0) x.set(victim, -1);
      x.set(e, s);
      if (lane == 0) {
        job_e[nm] = e;
        job_s[nm] = s;
        if (job_k) job_k[nm] = r;
      }
      if (lane == r) miss_r = true;
      ++nm;
    } else {
      ++hits;
    }
    if ((s & 63) == lane) touched |= 1u << (s >> 6);
    if (lane == r) slot_r = s;
  }
#pragma unroll
  for (int j = 0; j < PERC; ++j)
    if ((touched >> j) & 1u) t.st[j] = step;
}

// The device hit/miss counters, read when the kernel starts (with the other
// table loads) so that adding this call's counts at the end costs no
// memory round trip.
struct StatsPrefetch {
  int64_t hits = 0, misses = 0;
  __device__ __forceinline__ void load(const int64_t* stats) {
    if (stats) {
      hits = stats[0];
      misses = stats[1];
    }
  }
};

template <int PER>
__device__ __forceinline__ void resolve_finish(const SlotRegs<PER>& t, int64_t step, int32_t nm,
                                               int64_t hits, int32_t cap,
                                               int64_t* __restrict__ stamp,
                                               int64_t* __restrict__ step_ptr,
                                               int32_t* __restrict__ nmiss_ptr,
                                               int64_t* __restrict__ stats,
                                               const StatsPrefetch& prev) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = lane + 64 * j;
    if (c < cap) stamp[c] = t.st[j];
  }
  if (lane == 0) {
    *step_ptr = step;
    *nmiss_ptr = nm;
    if (stats) {
      stats[0] = prev.hits + hits;
      stats[1] = prev.misses + nm;
    }
  }
}

// General resolve of k ids from memory: id_at(i) -> id i (called by lane
// i%64 of chunk i/64); out-of-range ids are reported as slot -1.
template <int PER, typename IdAt>
__device__ __forceinline__ void resolve_wave_impl(IdAt id_at, int32_t k, int32_t n_experts,
                                                  int32_t* __restrict__ slot_of,
                                                  int32_t* __restrict__ slot_expert,
                                                  int64_t* __restrict__ stamp, int32_t cap,
                                                  int64_t* __restrict__ step_ptr,
                                                  int32_t* __restrict__ out_slot,
                                                  int32_t* __restrict__ fetch_slot,
                                                  int32_t* __restrict__ fetch_expert,
                                                  int32_t* __restrict__ nmiss_ptr,
                                                  int64_t* __restrict__ stats) {
  const int lane = threadIdx.x & 63;
  SlotRegs<PER> t;
  t.load(stamp, slot_expert, cap);
  StatsPrefetch prev;
  prev.load(stats);
  // read at run time, never a launch argument: a captured step would
  // otherwise stamp the same value on every replay
  const int64_t step = *step_ptr + 1;
  int32_t nm = 0;
  int64_t hits = 0;
  for (int32_t base = 0; base < k; base += 64) {
    int32_t my_e = -1, my_s = -1;
    if (base + lane < k) {
      my_e = id_at(base + lane);
      if (my_e >= 0 && my_e < n_experts)
        // coherent load: lane 0's writes of the previous chunk were fenced
        my_s = __hip_atomic_load(slot_of + my_e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        my_e = -1;
    }
    resolve_chunk<PER>(t, my_e, my_s, min(64, k - base), base, step, cap, slot_of, slot_expert,
                       out_slot, fetch_slot, fetch_expert, nm, hits);
    if (base + 64 < k) __threadfence();
  }
  resolve_finish<PER>(t, step, nm, hits, cap, stamp, step_ptr, nmiss_ptr, stats, prev);
}

}  // namespace moe
