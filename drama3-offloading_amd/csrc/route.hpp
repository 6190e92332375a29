// The decode router's top-k and the decode step's route (top-k + slot
// resolve on a double-buffered table by one wave), shared by the router
// kernels (router.hip), the decode step's fused launches (decode_step.hip,
// codec.hip) and the GEMV's gate/up launch when it makes the top-k itself
// (moe_gemv.hip).
#pragma once

#include "common.hpp"
#include "resolve.hpp"

namespace moe {

constexpr int kMaxTopK = 32;

// The decode router's logits launch (router.hip): one token's logits
// x . W^T rounded to bf16 (bf16_logits) or float32, + bias, into logits
// [n_experts]; adds one to *step_inc (nullable) for the route that follows
// and sets *ticket (nullable), the piece counter of its fetch, to zero.
int launch_decode_logits(const void* x, const void* w, const float* bias, int32_t hidden,
                         int32_t n_experts, int bf16_logits, float* logits, int64_t* step_inc,
                         hipStream_t s, int32_t* ticket = nullptr);

// The router's logits launch for `tokens` tokens (moe_router_topk's first
// launch): logits [tokens, n_experts].
int launch_router_logits(const void* x, const void* w, const float* bias, int32_t tokens,
                         int32_t hidden, int32_t n_experts, int bf16_logits, float* logits,
                         hipStream_t s);

// Order-preserving 32-bit key of a float logit: larger logit, larger key;
// NaN ranks below every number (it is picked only when nothing else is left).
__device__ __forceinline__ uint32_t logit_key(float f) {
  const uint32_t u = __float_as_uint(f);
  if (!(f == f)) return 1u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_logit(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Top-k of one token's logits by one wave.  Lane r < k ends up holding the
// r-th pick (*id, *wt = its renormalised softmax weight).  Each candidate is
// one 64-bit key, logit key above (~index) below, so a wave-wide max gives
// the largest logit with ties to the lower index.  Experts past n_experts
// get key 0 and are never picked (top_k <= n_experts).
//   PER <= 4: each lane sorts its keys once; a round takes the wave maximum
//             of the lanes' leading keys, and the winning lane (keys are
//             distinct) moves to its next key.
//   PER > 4:  a round takes the wave maximum of each lane's largest key,
//             which is then cleared.
// The weights are one exp per lane after the picks: exp(l_r - l_0) over
// their wave-wide sum.
// This lane's logits lane, lane + 64, ... of a row: every lane loads (past
// the end: the last logit again, then ignored), so the PER loads go out
// together; a load under the bound's branch would be waited for inside it,
// one memory round trip per load.
template <int PER>
__device__ __forceinline__ void load_logits(const float* __restrict__ row, int32_t n_experts,
                                            float (&lv)[PER]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < PER; ++j) lv[j] = row[min(lane + 64 * j, n_experts - 1)];
}

// The picks alone: lane r < k returns pick r's 64-bit key, (logit key << 32)
// | ~index (0 past k); topk_id and topk_weight turn it into the expert id
// and the renormalised softmax weight.
template <int PER>
__device__ __forceinline__ uint64_t wave_topk_keys(const float (&lv)[PER], int32_t n_experts,
                                                   int32_t top_k) {
  const int lane = threadIdx.x & 63;
  uint64_t key[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = lane + 64 * j;
    key[j] = e < n_experts
                 ? (static_cast<uint64_t>(logit_key(lv[j])) << 32) | (0xffffffffu - static_cast<uint32_t>(e))
                 : 0ull;
  }
  uint64_t pick = 0;
  if constexpr (PER <= 4) {
    // descending sorting network over the lane's PER keys
    auto cswap = [](uint64_t& a, uint64_t& b) {
      const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
      a = hi;
      b = lo;
    };
    if constexpr (PER == 2) cswap(key[0], key[1]);
    if constexpr (PER == 3) { cswap(key[0], key[1]); cswap(key[1], key[2]); cswap(key[0], key[1]); }
    if constexpr (PER == 4) {
      cswap(key[0], key[1]); cswap(key[2], key[3]);
      cswap(key[0], key[2]); cswap(key[1], key[3]);
      cswap(key[1], key[2]);
    }
    // A round's wave maximum of the lanes' leading keys, on 32-bit halves:
    // the largest logit key first; its index half read from the one lane
    // that holds it, or, when several lanes tie on the logit (bf16 logits
    // do), the largest index half among them (the lowest expert).  The
    // same key as the 64-bit maximum, for about a third of its
    // instructions.
    uint32_t hi[PER], lo[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      hi[j] = static_cast<uint32_t>(key[j] >> 32);
      lo[j] = static_cast<uint32_t>(key[j]);
    }
    for (int r = 0; r < top_k; ++r) {
      const uint32_t mh = wave_max_u32(hi[0]);
      const uint64_t tied = __builtin_amdgcn_ballot_w64(hi[0] == mh);
      const uint32_t ml =
          __builtin_popcountll(tied) == 1
              ? static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(lo[0]),
                                                                __builtin_ctzll(tied)))
              : wave_max_u32(hi[0] == mh ? lo[0] : 0u);
      if (lane == r) pick = (static_cast<uint64_t>(mh) << 32) | ml;
      if (hi[0] == mh && lo[0] == ml) {
#pragma unroll
        for (int j = 0; j + 1 < PER; ++j) {
          hi[j] = hi[j + 1];
          lo[j] = lo[j + 1];
        }
        hi[PER - 1] = lo[PER - 1] = 0u;
      }
    }
  } else {
    for (int r = 0; r < top_k; ++r) {
      uint64_t b = key[0];
#pragma unroll
      for (int j = 1; j < PER; ++j) b = key[j] > b ? key[j] : b;
      const uint64_t best = wave_reduce_u64<true>(b);
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (key[j] == best) key[j] = 0ull;
      if (lane == r) pick = best;
    }
  }
  return pick;
}

__device__ __forceinline__ int32_t topk_id(uint64_t pick, int32_t top_k) {
  const int lane = threadIdx.x & 63;
  return lane < top_k ? static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(pick)) : -1;
}

// exp(l_r - l_0) over the sum of the k picks' (a wave-wide call)
__device__ __forceinline__ float topk_weight(uint64_t pick, int32_t top_k) {
  const int lane = threadIdx.x & 63;
  const float v = key_logit(static_cast<uint32_t>(pick >> 32));
  const float m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float ex = lane < top_k ? expf(v - m) : 0.0f;
  return ex / wave_sum_f32_dpp(ex);
}

template <int PER>
__device__ __forceinline__ void wave_topk_of(const float (&lv)[PER], int32_t n_experts,
                                             int32_t top_k, int32_t* id, float* wt) {
  const uint64_t pick = wave_topk_keys<PER>(lv, n_experts, top_k);
  *id = topk_id(pick, top_k);
  *wt = topk_weight(pick, top_k);
}

template <int PER>
__device__ __forceinline__ void wave_topk(const float* __restrict__ row, int32_t n_experts,
                                          int32_t top_k, int32_t* id, float* wt) {
  float lv[PER];
  load_logits<PER>(row, n_experts, lv);
  wave_topk_of<PER>(lv, n_experts, top_k, id, wt);
}

// The decode step's route by the first wave of a workgroup (the other
// threads pass through): the top-k of one token's logits and the slot
// resolve (the decisions of topk_resolve_kernel) on the current buffer of a
// double-buffered table.  The call counted `step` (the logits launch before
// it adds one) reads buffer (step - 1) & 1; workgroup 0 writes ids,
// weights, out_slot, buffer step & 1, the fetch lists, nmiss and the
// counters.  Every workgroup makes the same decisions from the same inputs,
// none of which a workgroup of the launch writes, and gets the miss list in
// LDS: job_e / job_s (and job_k, the misses' positions in the top-k, when
// given), their count in *job_n.  Lane r of the first wave returns pick r's
// slot in slot_r and whether it missed in miss_r.  early(e) is called by
// the routing wave with the first miss's expert (first_miss) before the
// resolve, so that its caller can start reading that record.
struct NoEarly {
  __device__ void operator()(int32_t) const {}
};

// The expert of the route's first miss (-1 when every pick is in the
// table), known before the resolve: the picks ahead of the first one absent
// from the table are hits and evict nothing, so that one is the first miss
// and the resolve's job 0, whatever it decides for the picks after it.
// my_e: pick `lane` (-1 past top_k), my_s: its slot in the table (-1 absent).
__device__ __forceinline__ int32_t first_miss(int32_t my_e, int32_t my_s) {
  const uint64_t m = __builtin_amdgcn_ballot_w64(my_e >= 0 && my_s < 0);
  return m ? __builtin_amdgcn_readlane(my_e, __builtin_ctzll(m)) : -1;
}

template <int PER, int PERC, typename Early = NoEarly>
__device__ __forceinline__ void route_wave(
    const float* __restrict__ logits, int32_t n_experts, int32_t top_k,
    int32_t* __restrict__ ids, float* __restrict__ weights, int32_t* __restrict__ slot_of,
    int32_t* __restrict__ slot_expert, int64_t* __restrict__ stamp, int32_t cap,
    const int64_t* __restrict__ step_ptr, int32_t* __restrict__ out_slot,
    int32_t* __restrict__ fetch_slot, int32_t* __restrict__ fetch_expert,
    int32_t* __restrict__ nmiss_ptr, int64_t* __restrict__ stats, int32_t* job_e, int32_t* job_s,
    int32_t* job_k, int32_t* job_n, int32_t& slot_r, bool& miss_r, Early early = Early()) {
  slot_r = -1;
  miss_r = false;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    // both buffers, the step, the counters and the logits in one round trip
    SlotRegs<PERC> ta, tb;
    ta.load(stamp, slot_expert, cap);
    tb.load(stamp + cap, slot_expert + cap, cap);
    ExpertRegs<PER> xa, xb;
    xa.load(slot_of, n_experts);
    xb.load(slot_of + n_experts, n_experts);
    StatsPrefetch prev;
    prev.load(stats);
    int64_t step = *step_ptr;
    float lv[PER];
    load_logits<PER>(logits, n_experts, lv);
    // the step passes through this (empty) statement once every load above
    // is issued, so it is not loaded late, after the top-k
    asm volatile("" : "+s"(step));
    const uint64_t pick = wave_topk_keys<PER>(lv, n_experts, top_k);
    const int32_t id = topk_id(pick, top_k);
    const int cur = static_cast<int>((step - 1) & 1);
    SlotRegs<PERC> t;
    ExpertRegs<PER> x;
#pragma unroll
    for (int j = 0; j < PERC; ++j) {
      t.st[j] = cur ? tb.st[j] : ta.st[j];
      t.se[j] = cur ? tb.se[j] : ta.se[j];
    }
#pragma unroll
    for (int j = 0; j < PER; ++j) x.so[j] = cur ? xb.so[j] : xa.so[j];
    const int32_t my_e = lane < top_k ? id : -1;
    const int32_t found = x.lookup(my_e < 0 ? 0 : my_e);
    const int32_t my_s = my_e < 0 ? -1 : found;
    early(first_miss(my_e, my_s));
    const float wt = topk_weight(pick, top_k);
    int32_t nm = 0;
    int64_t hits = 0;
    resolve_regs<PER, PERC>(t, x, my_e, my_s, top_k, step, cap, job_e, job_s, job_k, nm, hits,
                            slot_r, miss_r);
    if (lane == 0) *job_n = nm;
    if (blockIdx.x == 0) {
      if (lane < top_k) {
        ids[lane] = id;
        weights[lane] = wt;
        out_slot[lane] = slot_r;
      }
      const int nxt = 1 - cur;
      int32_t* so_n = slot_of + static_cast<int64_t>(nxt) * n_experts;
      int32_t* se_n = slot_expert + static_cast<int64_t>(nxt) * cap;
      int64_t* st_n = stamp + static_cast<int64_t>(nxt) * cap;
#pragma unroll
      for (int j = 0; j < PERC; ++j) {
        const int c = lane + 64 * j;
        if (c < cap) {
          st_n[c] = t.st[j];
          se_n[c] = t.se[j];
        }
      }
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int e = lane + 64 * j;
        if (e < n_experts) so_n[e] = x.so[j];
      }
      if (lane == 0) {
        for (int j = 0; j < nm; ++j) {
          fetch_expert[j] = job_e[j];
          fetch_slot[j] = job_s[j];
        }
        *nmiss_ptr = nm;
        if (stats) {
          stats[0] = prev.hits + hits;
          stats[1] = prev.misses + nm;
        }
      }
    }
  }
}

// first_miss by a second wave of the route's workgroup, from the same
// inputs (the logits, the table's current slot_of, the counted step) as the
// routing wave; with UNCACHED, pick 0 (every pick misses).
template <int PER, bool UNCACHED>
__device__ __forceinline__ int32_t route_first_miss(const float* __restrict__ logits,
                                                    int32_t n_experts, int32_t top_k,
                                                    const int32_t* __restrict__ slot_of,
                                                    const int64_t* __restrict__ step_ptr) {
  const int lane = threadIdx.x & 63;
  ExpertRegs<PER> xa, xb;
  int64_t step = 0;
  if constexpr (!UNCACHED) {
    xa.load(slot_of, n_experts);
    xb.load(slot_of + n_experts, n_experts);
    step = *step_ptr;
  }
  float lv[PER];
  load_logits<PER>(logits, n_experts, lv);
  asm volatile("" : "+s"(step));
  const int32_t id = topk_id(wave_topk_keys<PER>(lv, n_experts, top_k), top_k);
  if constexpr (UNCACHED) {
    return __builtin_amdgcn_readlane(id, 0);
  } else {
    const int cur = static_cast<int>((step - 1) & 1);
    ExpertRegs<PER> x;
#pragma unroll
    for (int j = 0; j < PER; ++j) x.so[j] = cur ? xb.so[j] : xa.so[j];
    const int32_t my_e = lane < top_k ? id : -1;
    const int32_t found = x.lookup(my_e < 0 ? 0 : my_e);
    return first_miss(my_e, my_e < 0 ? -1 : found);
  }
}

// The uncached route by the first wave of a workgroup (the other threads
// pass through): the top-k of one token's logits, every pick a miss fetched
// into slot r (its position in the top-k), with no slot table: the
// reference's uncached per-expert transfer, every routed expert copied on
// every call (bin/offload.py:137-239).  The same LDS lists and per-lane
// returns as route_wave; workgroup 0 writes ids, weights, out_slot (= r),
// the fetch lists and nmiss (= top_k), and adds top_k misses to stats.
template <int PER, typename Early = NoEarly>
__device__ __forceinline__ void route_wave_uncached(
    const float* __restrict__ logits, int32_t n_experts, int32_t top_k,
    int32_t* __restrict__ ids, float* __restrict__ weights, int32_t* __restrict__ out_slot,
    int32_t* __restrict__ fetch_slot, int32_t* __restrict__ fetch_expert,
    int32_t* __restrict__ nmiss_ptr, int64_t* __restrict__ stats, int32_t* job_e,
    int32_t* job_s, int32_t* job_k, int32_t* job_n, int32_t& slot_r, bool& miss_r,
    Early early = Early()) {
  slot_r = -1;
  miss_r = false;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    StatsPrefetch prev;
    prev.load(stats);
    float lv[PER];
    load_logits<PER>(logits, n_experts, lv);
    const uint64_t pick = wave_topk_keys<PER>(lv, n_experts, top_k);
    const int32_t id = topk_id(pick, top_k);
    early(__builtin_amdgcn_readlane(id, 0));   // pick 0 is job 0
    const float wt = topk_weight(pick, top_k);
    if (lane < top_k) {
      job_e[lane] = id;
      job_s[lane] = lane;
      if (job_k) job_k[lane] = lane;
      slot_r = lane;
      miss_r = true;
    }
    if (lane == 0) *job_n = top_k;
    if (blockIdx.x == 0) {
      if (lane < top_k) {
        ids[lane] = id;
        weights[lane] = wt;
        out_slot[lane] = lane;
        fetch_expert[lane] = id;
        fetch_slot[lane] = lane;
      }
      if (lane == 0) {
        *nmiss_ptr = top_k;
        if (stats) {
          stats[0] = prev.hits;
          stats[1] = prev.misses + top_k;
        }
      }
    }
  }
}

}  // namespace moe
