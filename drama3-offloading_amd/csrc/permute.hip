// Token -> expert grouping (permute), its inverse (unpermute), and the
// torch.unique-style renumbering the reference uses for its gathered subsets.
//
// permute (n_experts > 1024; permute_fast_kernel below otherwise): one
// workgroup, O(pairs) work, stable and deterministic:
//   1. histogram of expert ids in LDS (atomic adds; counts do not depend on
//      the order they land in);
//   2. block-wide exclusive scan -> offsets, and a cursor per expert;
//   3. pairs are placed in rounds of 512 in pair order.  In a round, each
//      wave ranks its lanes among the lanes with the same expert (bit-sliced
//      ballot matching, one ballot per bit of the id), the per-wave
//      counts of an expert are packed as 7-bit fields of one 64-bit LDS word
//      (8 waves x at most 64), so a lane's position is
//        cursor[e] + (counts of e in earlier waves) + (rank in its wave)
//      -- exactly its rank in a stable sort -- and the expert's cursor then
//      advances by the round's total.
// No memory has to be cleared beforehand (nothing to memset in a graph).
#include "common.hpp"
#include "grouped.hpp"

namespace moe {

constexpr int kPermThreads = 1024;     // unique_inverse
constexpr int kPermMaxExperts = 4096;
constexpr int kPermPer = kPermMaxExperts / kPermThreads;
constexpr int kPlaceThreads = 512;     // permute: 8 waves, 7-bit count fields in a uint64
constexpr int kPlacePer = kPermMaxExperts / kPlaceThreads;
constexpr int kHoldRounds = 8;         // placement rounds whose ids stay in registers

__device__ __forceinline__ int32_t read_id(const void* ids, int ids64, int64_t p) {
  return ids64 ? static_cast<int32_t>(reinterpret_cast<const int64_t*>(ids)[p])
               : reinterpret_cast<const int32_t*>(ids)[p];
}

// Exclusive scan over the NW * 64 threads' values, returns the total.
template <int NW>
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
  if (tid < NW) {
    int32_t w = scratch[tid];
    int32_t wi = w;
#pragma unroll
    for (int o = 1; o < NW; o <<= 1) {
      int32_t n = __shfl_up(wi, o, 64);
      if (tid >= o) wi += n;
    }
    scratch[16 + tid] = wi - w;    // exclusive wave offsets
    if (tid == NW - 1) scratch[32] = wi;
  }
  __syncthreads();
  *out_prefix = scratch[16 + wave] + incl - v;
  int32_t total = scratch[32];
  __syncthreads();
  return total;
}

// Stable rank of a lane among the lanes of its wave holding the same expert
// e (e < 0: none), and the number of such lanes.  The match mask is the AND,
// over the bits of the id, of the ballot of that bit or of its complement:
// one ballot per id bit rather than one pass per distinct expert.
__device__ __forceinline__ void wave_match_rank(int32_t e, int nbits, uint64_t below_lane,
                                                int& rank, int& count) {
  uint64_t m = __ballot(e >= 0);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t bb = __ballot(bit);
    m &= bit ? bb : ~bb;
  }
  rank = __popcll(m & below_lane);
  count = __popcll(m);
}

__global__ __launch_bounds__(kPlaceThreads) void permute_kernel(
    const void* __restrict__ ids, int ids64, int64_t P, int32_t n_experts,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ sorted_pairs,
    int32_t* __restrict__ pair_pos, int32_t* __restrict__ tiles, int32_t* __restrict__ n_tiles,
    int32_t tile_tokens, QuantRowsJob quant) {
  __shared__ int32_t cursor[kPermMaxExperts];
  __shared__ uint64_t fields[kPermMaxExperts];
  __shared__ int32_t scratch[40];
  const int tid = threadIdx.x;
  if (blockIdx.x > 0) {
    // the activation rows, two tokens per workgroup (a 256-thread half each,
    // whole waves), beside workgroup 0's permutation; no barrier here
    const int64_t t = 2 * static_cast<int64_t>(blockIdx.x - 1) + (tid >> 8);
    if (t < quant.tokens) quant_row(quant, t, tid & 255);
    return;
  }
  const int lane = tid & 63, wave = tid >> 6;
  // ids of the first kHoldRounds rounds, read once with all loads in flight
  // (-1: id out of range, -2: past the last pair)
  int32_t held[kHoldRounds];
#pragma unroll
  for (int r = 0; r < kHoldRounds; ++r) held[r] = -2;
  if (P > 0) {
#pragma unroll
    for (int r = 0; r < kHoldRounds; ++r) {
      const int64_t p = static_cast<int64_t>(r) * kPlaceThreads + tid;
      const int32_t e = read_id(ids, ids64, p < P ? p : P - 1);
      held[r] = p < P ? ((e >= 0 && e < n_experts) ? e : -1) : -2;
    }
  }
  for (int e = tid; e < n_experts; e += kPlaceThreads) {
    cursor[e] = 0;
    fields[e] = 0;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kHoldRounds; ++r)
    if (held[r] >= 0) atomicAdd(&cursor[held[r]], 1);
  for (int64_t p = static_cast<int64_t>(kHoldRounds) * kPlaceThreads + tid; p < P;
       p += kPlaceThreads) {
    const int32_t e = read_id(ids, ids64, p);
    if (e >= 0 && e < n_experts) atomicAdd(&cursor[e], 1);
  }
  __syncthreads();
  // thread t owns the contiguous experts [t*PER, t*PER + PER) for the scan
  int32_t mine[kPlacePer];
  int32_t sum = 0;
#pragma unroll
  for (int j = 0; j < kPlacePer; ++j) {
    const int x = tid * kPlacePer + j;
    mine[j] = x < n_experts ? cursor[x] : 0;
    sum += mine[j];
  }
  int32_t base;
  const int32_t total = block_exclusive_scan<kPlaceThreads / 64>(sum, scratch, &base);
#pragma unroll
  for (int j = 0; j < kPlacePer; ++j) {
    const int x = tid * kPlacePer + j;
    if (x < n_experts) {
      counts[x] = mine[j];
      offsets[x] = base;
      cursor[x] = base;            // becomes the placement cursor
    }
    base += mine[j];
  }
  if (tid == 0) offsets[n_experts] = total;
  if (tiles) {
    // work tiles of the grouped kernels: (expert, first row of the segment)
    // for every tile_tokens rows of every expert's segment, in expert order
    int32_t nt[kPlacePer];
    int32_t tsum = 0;
#pragma unroll
    for (int j = 0; j < kPlacePer; ++j) {
      nt[j] = (mine[j] + tile_tokens - 1) / tile_tokens;
      tsum += nt[j];
    }
    int32_t tbase;
    const int32_t ttotal = block_exclusive_scan<kPlaceThreads / 64>(tsum, scratch, &tbase);
#pragma unroll
    for (int j = 0; j < kPlacePer; ++j) {
      const int x = tid * kPlacePer + j;
      for (int32_t i = 0; i < nt[j]; ++i) {
        tiles[2 * (tbase + i)] = x;
        tiles[2 * (tbase + i) + 1] = i * tile_tokens;
      }
      tbase += nt[j];
    }
    if (tid == 0) *n_tiles = ttotal;
  }
  __syncthreads();
  const uint64_t below_lane = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int nbits = n_experts > 1 ? 32 - __clz(n_experts - 1) : 0;
  // one round: pairs r0 + [0, 512), e the (held) expert code of pair r0 + tid
  auto place = [&](int64_t r0, int32_t e) {
    const int64_t p = r0 + tid;
    if (e == -1) pair_pos[p] = -1;             // no such expert: no position
    int rank, wcount;
    wave_match_rank(e, nbits, below_lane, rank, wcount);
    const bool first = e >= 0 && rank == 0;    // one lane per (wave, expert)
    if (first) atomicAdd(reinterpret_cast<unsigned long long*>(&fields[e]),
                         static_cast<unsigned long long>(wcount) << (7 * wave));
    __syncthreads();
    uint64_t f = 0;
    if (e >= 0) {
      f = fields[e];
      int32_t before = 0;
      for (int w = 0; w < wave; ++w) before += static_cast<int32_t>((f >> (7 * w)) & 0x7f);
      const int32_t pos = cursor[e] + before + rank;
      sorted_pairs[pos] = static_cast<int32_t>(p);
      pair_pos[p] = pos;
    }
    __syncthreads();
    // the lowest wave holding expert e advances its cursor and clears its word
    if (first && (f & ((1ull << (7 * wave)) - 1ull)) == 0ull) {
      int32_t tot = 0;
#pragma unroll
      for (int w = 0; w < kPlaceThreads / 64; ++w) tot += static_cast<int32_t>((f >> (7 * w)) & 0x7f);
      cursor[e] += tot;
      fields[e] = 0;
    }
    __syncthreads();
  };
  const int64_t n_rounds = (P + kPlaceThreads - 1) / kPlaceThreads;
#pragma unroll
  for (int r = 0; r < kHoldRounds; ++r)
    if (r < n_rounds) place(static_cast<int64_t>(r) * kPlaceThreads, held[r]);
  for (int64_t r = kHoldRounds; r < n_rounds; ++r) {
    const int64_t p = r * kPlaceThreads + tid;
    int32_t e = -2;
    if (p < P) {
      e = read_id(ids, ids64, p);
      if (e < 0 || e >= n_experts) e = -1;
    }
    place(r * kPlaceThreads, e);
  }
}

// permute for n_experts <= kFastExperts: 16 waves, and 4096 pairs per
// placement pass instead of 512, so one pass serves a 512-token top-8 call.
// Wave w takes pairs [4096c + 256w, +256) of pass c in 4 rounds of 64 (lane
// l of round j: pair 4096c + 256w + 64j + l).  In a round each lane finds
// the lanes of its expert (ballot matching, as above); its rank in the wave
// is the wave's count of that expert from earlier rounds, kept in LDS as one
// 16-bit word per (wave, expert) and advanced by the expert's lowest lane,
// plus its rank in the round.  Then one thread per expert turns the 16
// waves' counts into exclusive prefixes, and a pair's position is
//   cursor[e] + (its wave's prefix) + (its rank in the wave)
// -- its rank in a stable sort.  Four barriers per pass.
constexpr int kFastThreads = 1024;
constexpr int kFastWaves = kFastThreads / 64;
constexpr int kFastRounds = 4;
constexpr int kFastPass = kFastThreads * kFastRounds;   // pairs per placement pass
constexpr int kFastExperts = 1024;                      // one thread per expert

__global__ __launch_bounds__(kFastThreads) void permute_fast_kernel(
    const void* __restrict__ ids, int ids64, int64_t P, int32_t n_experts,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ sorted_pairs,
    int32_t* __restrict__ pair_pos, int32_t* __restrict__ tiles, int32_t* __restrict__ n_tiles,
    int32_t tile_tokens, QuantRowsJob quant) {
  __shared__ int32_t cursor[kFastExperts];
  __shared__ uint16_t wcount[kFastWaves * kFastExperts];   // [wave][expert]
  __shared__ int32_t scratch[40];
  const int tid = threadIdx.x;
  if (blockIdx.x > 0) {
    // the activation rows, four tokens per workgroup (a 256-thread quarter
    // each, whole waves), beside workgroup 0's permutation; no barrier here
    const int64_t t = 4 * static_cast<int64_t>(blockIdx.x - 1) + (tid >> 8);
    if (t < quant.tokens) quant_row(quant, t, tid & 255);
    return;
  }
  const int lane = tid & 63, wave = tid >> 6;
  const int E = n_experts;
  // expert codes of this lane's pairs in a pass (-1: id out of range, -2:
  // past the last pair)
  auto load_pass = [&](int64_t c0, int32_t (&e)[kFastRounds]) {
#pragma unroll
    for (int j = 0; j < kFastRounds; ++j) {
      const int64_t p = c0 + wave * (64 * kFastRounds) + j * 64 + lane;
      const int32_t v = read_id(ids, ids64, p < P ? p : P - 1);
      e[j] = p < P ? ((v >= 0 && v < E) ? v : -1) : -2;
    }
  };
  int32_t held[kFastRounds];
#pragma unroll
  for (int j = 0; j < kFastRounds; ++j) held[j] = -2;
  if (P > 0) load_pass(0, held);
  if (tid < E) {
    cursor[tid] = 0;
#pragma unroll
    for (int w = 0; w < kFastWaves; ++w) wcount[w * kFastExperts + tid] = 0;
  }
  __syncthreads();
  // histogram (LDS atomics; the counts do not depend on the order)
#pragma unroll
  for (int j = 0; j < kFastRounds; ++j)
    if (held[j] >= 0) atomicAdd(&cursor[held[j]], 1);
  for (int64_t p = kFastPass + tid; p < P; p += kFastThreads) {
    const int32_t v = read_id(ids, ids64, p);
    if (v >= 0 && v < E) atomicAdd(&cursor[v], 1);
  }
  __syncthreads();
  // thread t owns expert t: counts, offsets, and the placement cursor
  const int32_t mine = tid < E ? cursor[tid] : 0;
  int32_t base;
  const int32_t total = block_exclusive_scan<kFastWaves>(mine, scratch, &base);
  if (tid < E) {
    counts[tid] = mine;
    offsets[tid] = base;
    cursor[tid] = base;
  }
  if (tid == 0) offsets[E] = total;
  if (tiles) {
    // work tiles of the grouped kernels: (expert, first row of the segment)
    // for every tile_tokens rows of every expert's segment, in expert order
    const int32_t nt = (mine + tile_tokens - 1) / tile_tokens;
    int32_t tbase;
    const int32_t ttotal = block_exclusive_scan<kFastWaves>(nt, scratch, &tbase);
    for (int32_t i = 0; i < nt; ++i) {
      tiles[2 * (tbase + i)] = tid;
      tiles[2 * (tbase + i) + 1] = i * tile_tokens;
    }
    if (tid == 0) *n_tiles = ttotal;
  }
  __syncthreads();
  const uint64_t below_lane = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 0;
  uint16_t* wc = wcount + wave * kFastExperts;
  for (int64_t c0 = 0; c0 < P; c0 += kFastPass) {
    if (c0 > 0) load_pass(c0, held);
    // rank of each pair among its wave's pairs of the same expert
    int32_t rank[kFastRounds];
#pragma unroll
    for (int j = 0; j < kFastRounds; ++j) {
      const int32_t e = held[j];
      int r, n;
      wave_match_rank(e, nbits, below_lane, r, n);
      const int32_t prior = e >= 0 ? wc[e] : 0;    // earlier rounds of this wave
      rank[j] = prior + r;
      if (e >= 0 && r == 0) wc[e] = static_cast<uint16_t>(prior + n);
    }
    __syncthreads();
    // per expert: the waves' counts -> exclusive prefixes, and the pass total
    int32_t pass_total = 0;
    if (tid < E) {
      uint16_t v[kFastWaves];
#pragma unroll
      for (int w = 0; w < kFastWaves; ++w) v[w] = wcount[w * kFastExperts + tid];
#pragma unroll
      for (int w = 0; w < kFastWaves; ++w) {
        wcount[w * kFastExperts + tid] = static_cast<uint16_t>(pass_total);
        pass_total += v[w];
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kFastRounds; ++j) {
      const int64_t p = c0 + wave * (64 * kFastRounds) + j * 64 + lane;
      const int32_t e = held[j];
      if (e >= 0) {
        const int32_t pos = cursor[e] + wc[e] + rank[j];
        sorted_pairs[pos] = static_cast<int32_t>(p);
        pair_pos[p] = pos;
      } else if (e == -1) {
        pair_pos[p] = -1;                        // no such expert: no position
      }
    }
    __syncthreads();
    // the next pass starts after this one's pairs, with its counts cleared
    if (tid < E) {
      cursor[tid] += pass_total;
#pragma unroll
      for (int w = 0; w < kFastWaves; ++w) wcount[w * kFastExperts + tid] = 0;
    }
    __syncthreads();
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
    int32_t tot = block_exclusive_scan<kPermThreads / 64>(present, scratch, &pre);
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

// out[t][c] = sum_k w[t][k] * y[pair_pos[t*K+k]][c], k in order -> bf16.
// Each term is one explicit fused multiply-add, acc = fma(w, y, acc), which
// is exactly the combine of the per-pair GEMV path, so both paths give
// bit-identical outputs.
__global__ __launch_bounds__(256) void unpermute_kernel(const float* __restrict__ y,
                                                        const int32_t* __restrict__ pair_pos,
                                                        const void* __restrict__ weights,
                                                        int wbf16, int32_t top_k, int32_t hidden,
                                                        const uint16_t* __restrict__ residual,
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
    acc.x = fmaf(w, v.x, acc.x);
    acc.y = fmaf(w, v.y, acc.y);
    acc.z = fmaf(w, v.z, acc.z);
    acc.w = fmaf(w, v.w, acc.w);
  }
  uint16_t v[4] = {f32_to_bf16(acc.x), f32_to_bf16(acc.y), f32_to_bf16(acc.z),
                   f32_to_bf16(acc.w)};
  if (residual) {   // a bf16 tensor add: bf16(res + bf16(moe))
    const uint16_t* r = residual + t * hidden + c;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = f32_to_bf16(bf16_to_f32(r[i]) + bf16_to_f32(v[i]));
  }
  uint16_t* o = out + t * hidden + c;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = v[i];
}

// Hybrid prefill gather plan: the distinct experts uniq[0..n) of a call are
// split between those resident in the device cache (copied device to device
// from their slot) and the rest (fetched from the host pool), both lists in
// uniq order.  The table is only read: no stamp, no insert.  One wave; the
// lists are compacted with ballots, so the result is deterministic.
__global__ __launch_bounds__(64) void gather_plan_kernel(
    const int32_t* __restrict__ uniq, const int32_t* __restrict__ n_unique,
    const int32_t* slot_of, int32_t n_experts, int32_t cap,
    int32_t* __restrict__ host_expert, int32_t* __restrict__ host_dst, int32_t* __restrict__ n_host,
    int32_t* __restrict__ cache_src, int32_t* __restrict__ cache_dst,
    int32_t* __restrict__ n_cache, int64_t* __restrict__ stats) {
  const int lane = threadIdx.x;
  const int n = min(max(*n_unique, 0), n_experts);
  int nh = 0, nc = 0;
  for (int base = 0; base < n; base += 64) {
    const int i = base + lane;
    const int32_t e = i < n ? uniq[i] : -1;
    const bool valid = e >= 0 && e < n_experts;
    const int32_t s = valid && slot_of ? slot_of[e] : -1;   // no cache: all from host
    const bool cached = valid && s >= 0 && s < cap;
    const bool host = valid && !cached;
    const uint64_t mc = __ballot(cached);
    const uint64_t mh = __ballot(host);
    const int rc = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mc >> 32),
                                             __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mc), 0));
    const int rh = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mh >> 32),
                                             __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mh), 0));
    if (cached) {
      cache_src[nc + rc] = s;
      cache_dst[nc + rc] = i;
    }
    if (host) {
      host_expert[nh + rh] = e;
      host_dst[nh + rh] = i;
    }
    nc += __popcll(mc);
    nh += __popcll(mh);
  }
  if (lane == 0) {
    *n_host = nh;
    *n_cache = nc;
    if (stats) {
      stats[0] += nc;
      stats[1] += nh;
    }
  }
}

int launch_permute(const void* ids, int ids64, int64_t P, int32_t n_experts, int32_t* counts,
                   int32_t* offsets, int32_t* sorted_pairs, int32_t* pair_pos, hipStream_t s,
                   int32_t* tiles, int32_t* n_tiles, int32_t tile_tokens,
                   const QuantRowsJob* quant) {
  static_assert(kPlaceThreads == 512, "two 256-thread token slices per quantising workgroup");
  static_assert(kFastThreads == 1024, "four 256-thread token slices per quantising workgroup");
  const QuantRowsJob q = quant ? *quant : QuantRowsJob{nullptr, 0, nullptr, nullptr, 0};
  if (n_experts <= kFastExperts) {
    const unsigned grid = 1 + static_cast<unsigned>((q.tokens + 3) / 4);
    hipLaunchKernelGGL(permute_fast_kernel, dim3(grid), dim3(kFastThreads), 0, s, ids, ids64, P,
                       n_experts, counts, offsets, sorted_pairs, pair_pos, tiles, n_tiles,
                       tile_tokens, q);
  } else {
    const unsigned grid = 1 + static_cast<unsigned>((q.tokens + 1) / 2);
    hipLaunchKernelGGL(permute_kernel, dim3(grid), dim3(kPlaceThreads), 0, s, ids, ids64, P,
                       n_experts, counts, offsets, sorted_pairs, pair_pos, tiles, n_tiles,
                       tile_tokens, q);
  }
  return check_launch("moe_permute");
}

int launch_unpermute(const float* y, const int32_t* pair_pos, const void* weights, int wbf16,
                     int32_t tokens, int32_t top_k, int32_t hidden, const uint16_t* residual,
                     uint16_t* out, hipStream_t s) {
  hipLaunchKernelGGL(unpermute_kernel, dim3((hidden / 4 + 255) / 256, tokens), dim3(256), 0, s,
                     y, pair_pos, weights, wbf16, top_k, hidden, residual, out);
  return check_launch("moe_unpermute");
}

}  // namespace moe

using namespace moe;

extern "C" int moe_permute(const void* ids, int32_t ids_dtype, int32_t tokens, int32_t top_k,
                           int32_t n_experts, int32_t* counts, int32_t* offsets,
                           int32_t* sorted_pairs, int32_t* pair_pos, void* stream) {
  MOE_REQUIRE(ids_dtype == MOE_I32 || ids_dtype == MOE_I64, "moe_permute: bad ids_dtype");
  MOE_REQUIRE(tokens >= 0 && top_k >= 1, "moe_permute: need tokens >= 0, top_k >= 1");
  MOE_REQUIRE(n_experts >= 1 && n_experts <= kPermMaxExperts,
              "moe_permute: need 1 <= n_experts <= %d", kPermMaxExperts);
  const int64_t P = static_cast<int64_t>(tokens) * top_k;
  // no pairs: counts and offsets are still written (all zero); the per-pair
  // arrays may be NULL
  MOE_REQUIRE(counts && offsets && (P == 0 || (ids && sorted_pairs && pair_pos)),
              "moe_permute: NULL pointer");
  MOE_REQUIRE(P <= (1LL << 24), "moe_permute: too many pairs (%lld)", (long long)P);
  return launch_permute(ids, ids_dtype == MOE_I64 ? 1 : 0, P, n_experts, counts, offsets,
                        sorted_pairs, pair_pos, as_stream(stream));
}

extern "C" int moe_unique_inverse(const void* ids, int32_t ids_dtype, int32_t tokens,
                                  int32_t top_k, int32_t n_experts, const int32_t* counts,
                                  int32_t* n_unique, int32_t* uniq, int32_t* rank_of,
                                  int32_t* inverse, void* stream) {
  MOE_REQUIRE(ids_dtype == MOE_I32 || ids_dtype == MOE_I64, "moe_unique_inverse: bad ids_dtype");
  MOE_REQUIRE(tokens >= 0 && top_k >= 1, "moe_unique_inverse: need tokens >= 0, top_k >= 1");
  MOE_REQUIRE(n_experts >= 1 && n_experts <= kPermMaxExperts,
              "moe_unique_inverse: need 1 <= n_experts <= %d", kPermMaxExperts);
  const int64_t P = static_cast<int64_t>(tokens) * top_k;
  MOE_REQUIRE(counts && n_unique && uniq && rank_of && (P == 0 || (ids && inverse)),
              "moe_unique_inverse: NULL pointer");
  hipLaunchKernelGGL(unique_inverse_kernel, dim3(1), dim3(kPermThreads), 0, as_stream(stream), ids,
                     ids_dtype == MOE_I64 ? 1 : 0, P, n_experts, counts, n_unique, uniq, rank_of,
                     inverse);
  return check_launch("moe_unique_inverse");
}

extern "C" int moe_unpermute(const float* y, const int32_t* pair_pos, const void* weights,
                             int32_t w_dtype, int32_t tokens, int32_t top_k, int32_t hidden,
                             void* out, void* stream) {
  MOE_REQUIRE(w_dtype == MOE_F32 || w_dtype == MOE_BF16, "moe_unpermute: bad w_dtype");
  MOE_REQUIRE(tokens >= 0 && top_k >= 1, "moe_unpermute: need tokens >= 0, top_k >= 1");
  MOE_REQUIRE(hidden > 0 && hidden % 4 == 0, "moe_unpermute: hidden %% 4 != 0");
  if (tokens == 0) return MOE_OK;
  MOE_REQUIRE(y && pair_pos && weights && out, "moe_unpermute: NULL pointer");
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(y) % 16 == 0, "moe_unpermute: y must be 16-byte aligned");
  return launch_unpermute(y, pair_pos, weights, w_dtype == MOE_BF16 ? 1 : 0, tokens, top_k,
                          hidden, nullptr, static_cast<uint16_t*>(out), as_stream(stream));
}

extern "C" int moe_gather_plan(const int32_t* uniq, const int32_t* n_unique,
                               const int32_t* slot_of, int32_t n_experts, int32_t cap,
                               int32_t* host_expert, int32_t* host_dst, int32_t* n_host,
                               int32_t* cache_src, int32_t* cache_dst, int32_t* n_cache,
                               int64_t* stats, void* stream) {
  MOE_REQUIRE(uniq && n_unique && host_expert && host_dst && n_host && cache_src && cache_dst &&
                  n_cache, "moe_gather_plan: NULL pointer");
  MOE_REQUIRE(n_experts >= 1 && n_experts <= kPermMaxExperts,
              "moe_gather_plan: need 1 <= n_experts <= %d", kPermMaxExperts);
  MOE_REQUIRE(cap >= 0 && (cap == 0 || slot_of), "moe_gather_plan: cap > 0 needs slot_of");
  if (cap == 0) slot_of = nullptr;   // no device cache: every expert from the host
  hipLaunchKernelGGL(gather_plan_kernel, dim3(1), dim3(64), 0, as_stream(stream), uniq, n_unique,
                     slot_of, n_experts, cap, host_expert, host_dst, n_host, cache_src, cache_dst,
                     n_cache, stats);
  return check_launch("moe_gather_plan");
}
