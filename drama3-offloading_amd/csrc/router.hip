// Top-k-of-E router: logits = x . W^T (+ bias), top-k by descending logit
// (ties to the lower expert), softmax over the k selected (== softmax over all
// E then renormalise, upstream's norm_topk_prob).
//
// Logit arithmetic: a bf16 x bf16 product is exact in float32; products are
// summed in float64 and rounded once, to float32 or (the gate of a bf16
// nn.Linear, whose output is a bf16 tensor) to bf16, before the optional
// float32 bias.  With float64 partial sums exact for ordinary data, the
// rounded logit does not depend on the order of summation, which is what
// lets expert ids match the oracle bit for bit.
//
// Kernels:
//   logits: grid (E, ceil(T/TB)) of one wave, TB = 1 for one token else 4;
//           the wave of workgroup (bx, by) computes expert bx for the TB
//           tokens of block by, reading its 4 KiB gate row once.
//   topk:   one wave per token, logits in registers, k rounds of a wave-wide
//           max of (logit, ~index) keys (DPP, no LDS shuffles).
//   topk_resolve (decode): one wave does the top-k of one token AND the slot
//           table update for those ids (slots.hip's resolve, same decisions),
//           saving a launch per layer on the decode step.
// Cross-workgroup hand-offs happen only at kernel boundaries: on MI355X each
// XCD has its own L2, and a device-scope fence inside a kernel costs more
// than a launch.
#include "common.hpp"
#include "fetch.hpp"
#include "resolve.hpp"
#include "route.hpp"

namespace moe {

constexpr int kTokBlock = 4;     // tokens per logits workgroup when tokens > 1
// Experts (one per wave) per logits workgroup: one-wave workgroups spread the
// gate rows over every CU.  The decode router's two launches measured
// 8.95 us per call at 1 or 2, 9.10 at 4 (a graph over 40 gates, MI355X).
constexpr int kLogitWaves = 1;

// Wave-wide float64 sum, uniform in every lane: DPP butterfly inside each
// row of 16 lanes, then the four row sums read as scalars and added in row
// order.  The products summed here are exact and their float64 partial sums
// are exact for ordinary data, so the order does not change the result.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = __double_as_longlong(v);
  const uint32_t lo = __builtin_amdgcn_update_dpp(0u, static_cast<uint32_t>(u), CTRL, 0xf, 0xf,
                                                  true);
  const uint32_t hi = __builtin_amdgcn_update_dpp(0u, static_cast<uint32_t>(u >> 32), CTRL, 0xf,
                                                  0xf, true);
  return __longlong_as_double(static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo));
}

__device__ __forceinline__ double wave_sum_f64_dpp(double v) {
  v += dpp_f64<0x0B1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f64<0x04E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f64<0x141>(v);   // row_half_mirror
  v += dpp_f64<0x140>(v);   // row_mirror
  const uint64_t u = __double_as_longlong(v);
  double s = 0.0;
#pragma unroll
  for (int row = 0; row < 4; ++row) {
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(u)), row * 16);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(u >> 32)), row * 16);
    s += __longlong_as_double(static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo));
  }
  return s;
}

// bf16 (round to nearest, ties to even) of a double, returned as a float.
// The double is first rounded to odd into float32 (toward zero, then the
// last bit set when anything was dropped); float32 keeps 24 significant
// bits, at least two more than bf16's 8, so rounding that result to nearest
// even gives the correctly rounded bf16 of the double itself.
__device__ __forceinline__ float bf16_of_f64(double s) {
  const float f = __double2float_rz(s);
  uint32_t u = __float_as_uint(f);
  if (static_cast<double>(f) != s) u |= 1u;
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  return __uint_as_float(u);
}

// One wave per (expert, block of TB tokens): the expert's gate row and the
// tokens' rows are read in chunks of 4 x 16 bytes per lane, every load of a
// chunk issued before any of it is used (no load under a branch: lanes and
// tokens past the end re-read an in-bounds address and add nothing).
template <int TB>
__global__ __launch_bounds__(64 * kLogitWaves) void router_logits_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const float* __restrict__ bias,
    int32_t tokens, int32_t hidden, int32_t n_experts, int bf16_logits,
    float* __restrict__ logits, int64_t* __restrict__ step_inc, int32_t* __restrict__ ticket) {
  constexpr int U = 4;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  // No early exit for a wave past the last expert (it computes the last
  // expert's logit again and stores nothing): a branch on n_experts would
  // wait for that argument before the other arguments are even requested.
  const int e_raw = blockIdx.x * kLogitWaves + wave;
  const bool live = e_raw < n_experts;
  const int e = live ? e_raw : n_experts - 1;
  const int t0 = blockIdx.y * TB;
  const int nt = min(TB, tokens - t0);
  const int nv = hidden >> 3;                 // 16-byte vectors per row
  const uint4* wr = reinterpret_cast<const uint4*>(w + static_cast<int64_t>(e) * hidden);
  const uint4* xr[TB];
#pragma unroll
  for (int tt = 0; tt < TB; ++tt)
    xr[tt] = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(t0 + min(tt, nt - 1)) * hidden);
  double acc[TB];
#pragma unroll
  for (int tt = 0; tt < TB; ++tt) acc[tt] = 0.0;
  uint4 b[U], a[TB][U];
  // chunk i0 of the row: 64 * U vectors, every lane's loads issued together
  // (lanes past the end re-read the last vector)
  auto load_chunk = [&](int i0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + 64 * u + lane;
      const int ic = i < nv ? i : nv - 1;
      b[u] = wr[ic];
#pragma unroll
      for (int tt = 0; tt < TB; ++tt) a[tt][u] = xr[tt][ic];
    }
  };
  // Lanes past the end add +0.0, which leaves a partial sum as it is (a sum
  // that starts at +0.0 never becomes -0.0).  No branch: under a lane
  // condition the compiler moved a chunk's first loads into the branch and
  // waited for each there.
  auto add_chunk = [&](int i0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool in = i0 + 64 * u + lane < nv;
      const uint32_t bv[4] = {b[u].x, b[u].y, b[u].z, b[u].w};
#pragma unroll
      for (int tt = 0; tt < TB; ++tt) {
        const uint32_t av[4] = {a[tt][u].x, a[tt][u].y, a[tt][u].z, a[tt][u].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a0 = __uint_as_float(av[j] << 16), a1 = __uint_as_float(av[j] & 0xffff0000u);
          const float b0 = __uint_as_float(bv[j] << 16), b1 = __uint_as_float(bv[j] & 0xffff0000u);
          acc[tt] += in ? static_cast<double>(a0 * b0) : 0.0;     // exact products
          acc[tt] += in ? static_cast<double>(a1 * b1) : 0.0;
        }
      }
    }
  };
  // The first chunk (the whole row up to hidden 2048) outside any loop, so
  // that no loop-carried wait holds its loads back; the bias goes out after
  // them (from the first word of the gate row when there is none, read and
  // ignored): loaded where it is added, it would put a memory round trip
  // after the sum.
  load_chunk(0);
  __builtin_amdgcn_sched_barrier(0);
  const float bias_raw = *(bias ? bias + e : reinterpret_cast<const float*>(wr));
  __builtin_amdgcn_sched_barrier(0);
  add_chunk(0);
  for (int i0 = 64 * U; i0 < nv; i0 += 64 * U) {
    load_chunk(i0);
    add_chunk(i0);
  }
#pragma unroll
  for (int tt = 0; tt < TB; ++tt) {
    const double s = wave_sum_f64_dpp(acc[tt]);
    if (lane == 0 && tt < nt && live) {
      float l = bf16_logits ? bf16_of_f64(s) : static_cast<float>(s);
      if (bias) l += bias_raw;
      logits[static_cast<int64_t>(t0 + tt) * n_experts + e] = l;
    }
  }
  // The route + fetch launch that follows reads the slot-table step already
  // counted, so that none of its workgroups writes what another one reads.
  // An atomic add whose result is unused waits for nothing (a load and a
  // store would add a memory round trip), and at the end it holds no
  // argument loads back either.
  if (step_inc && e_raw == 0 && blockIdx.y == 0 && lane == 0)
    __hip_atomic_fetch_add(step_inc, int64_t{1}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // ... and finds the counter its fetch waves take pieces from at zero
  if (ticket && e_raw == 0 && blockIdx.y == 0 && lane == 0) *ticket = 0;
}

// Many tokens: the logits on the float64 matrix cores.  A workgroup takes 16
// experts x 16 tokens; its kLogitMmaWaves waves split K, wave v taking the
// 32-wide chunks v, v + kLogitMmaWaves, ...  Lane (q, i) = (lane / 16, lane %
// 16) loads 16 bytes of expert i's gate row and of token i's row, K 8q ..
// 8q + 7 of a chunk, and each of its 8 bf16 pairs is one 16x16x4 float64
// MFMA (the lane group q's K index of every MFMA), so every product of the
// chunk is formed once, exact in float64.  The products are the vector
// kernel's, and so is the float64 sum wherever it is exact (ordinary
// data), whatever its order; the partial sums of the waves are added
// through LDS, and the logit is rounded as the vector kernel rounds it.
typedef double v4d __attribute__((ext_vector_type(4)));

// A 16 x 16 tile is 512 float64 MFMAs over H 2048, about 3.4 us of one CU's
// float64 matrix rate, so the form pays from the token count at which the
// vector kernel's per-token work exceeds that.  Measured on MI355X
// (moe_router_topk, 256 experts, H 2048, a graph over 40 gates): vector
// 8.2 / 9.9 / 12.7 / 15.5 / 18.2 / 28.6 / 50.5 us at 16 / 32 / 64 / 96 /
// 128 / 256 / 512 tokens, this form 12.0 up to 256 tokens and 19.2 at 512.
constexpr int kLogitMmaWaves = 8;       // K slices per workgroup
constexpr int kLogitMmaChunks = 8;      // 32-wide K chunks per wave in flight
constexpr int kLogitMmaFrom = 64;       // tokens from which this form runs

__device__ __forceinline__ double bf16_elem(u32x4 v, int m) {
  const uint32_t w = m < 2 ? v.x : m < 4 ? v.y : m < 6 ? v.z : v.w;
  return static_cast<double>(__uint_as_float((m & 1) ? (w & 0xffff0000u) : (w << 16)));
}

__global__ __launch_bounds__(64 * kLogitMmaWaves) void router_logits_mma_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const float* __restrict__ bias,
    int32_t tokens, int32_t hidden, int32_t n_experts, int bf16_logits,
    float* __restrict__ logits) {
  __shared__ double part[kLogitMmaWaves][16][17];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = lane & 15, q = lane >> 4;
  const int e0 = static_cast<int>(blockIdx.x) * 16, t0 = static_cast<int>(blockIdx.y) * 16;
  const uint16_t* wr = w + static_cast<int64_t>(min(e0 + i, n_experts - 1)) * hidden + 8 * q;
  const uint16_t* xr = x + static_cast<int64_t>(min(t0 + i, tokens - 1)) * hidden + 8 * q;
  const int nchunk = hidden >> 5;
  v4d acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = v4d{0.0, 0.0, 0.0, 0.0};
  for (int c0 = wave; c0 < nchunk; c0 += kLogitMmaWaves * kLogitMmaChunks) {
    u32x4 a[kLogitMmaChunks], b[kLogitMmaChunks];
#pragma unroll
    for (int u = 0; u < kLogitMmaChunks; ++u) {
      const int64_t o = static_cast<int64_t>(min(c0 + u * kLogitMmaWaves, nchunk - 1)) * 32;
      a[u] = *reinterpret_cast<const u32x4*>(wr + o);
      b[u] = *reinterpret_cast<const u32x4*>(xr + o);
    }
    __builtin_amdgcn_sched_barrier(0);   // every load above is issued before the math below
#pragma unroll
    for (int u = 0; u < kLogitMmaChunks; ++u) {
      // a chunk past the end re-read the last one: zeros (no branch)
      const bool live = c0 + u * kLogitMmaWaves < nchunk;
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const double av = live ? bf16_elem(a[u], m) : 0.0;
        const double bv = live ? bf16_elem(b[u], m) : 0.0;
        acc[m & 3] = __builtin_amdgcn_mfma_f64_16x16x4f64(av, bv, acc[m & 3], 0, 0, 0);
      }
    }
  }
  // element r of lane (q, i) holds expert 4r + q of token column i (the
  // float64 MFMA's result layout)
#pragma unroll
  for (int r = 0; r < 4; ++r)
    part[wave][4 * r + q][i] = (acc[0][r] + acc[1][r]) + (acc[2][r] + acc[3][r]);
  __syncthreads();
  if (threadIdx.x < 256) {
    const int rr = threadIdx.x & 15, j = threadIdx.x >> 4;
    double sum = part[0][rr][j];
#pragma unroll
    for (int v = 1; v < kLogitMmaWaves; ++v) sum += part[v][rr][j];
    const int e = e0 + rr, t = t0 + j;
    if (e < n_experts && t < tokens) {
      float l = bf16_logits ? bf16_of_f64(sum) : static_cast<float>(sum);
      if (bias) l += bias[e];
      logits[static_cast<int64_t>(t) * n_experts + e] = l;
    }
  }
}

template <int PER>
__global__ __launch_bounds__(64) void router_topk_kernel(const float* __restrict__ logits,
                                                         int32_t n_experts, int32_t top_k,
                                                         void* __restrict__ ids, int ids64,
                                                         void* __restrict__ weights, int wbf16) {
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x;
  int32_t id;
  float wt;
  wave_topk<PER>(logits + t * n_experts, n_experts, top_k, &id, &wt);
  if (lane < top_k) {
    const int64_t o = t * top_k + lane;
    if (ids64) reinterpret_cast<int64_t*>(ids)[o] = id;
    else reinterpret_cast<int32_t*>(ids)[o] = id;
    if (wbf16) reinterpret_cast<uint16_t*>(weights)[o] = f32_to_bf16(wt);
    else reinterpret_cast<float*>(weights)[o] = wt;
  }
}

template <int PER, int PERC>
__global__ __launch_bounds__(64) void topk_resolve_kernel(
    const float* __restrict__ logits, int32_t n_experts, int32_t top_k, int32_t* __restrict__ ids,
    float* __restrict__ weights, int32_t* __restrict__ slot_of, int32_t* __restrict__ slot_expert,
    int64_t* __restrict__ stamp, int32_t cap, int64_t* __restrict__ step_ptr,
    int32_t* __restrict__ out_slot, int32_t* __restrict__ fetch_slot,
    int32_t* __restrict__ fetch_expert, int32_t* __restrict__ nmiss_ptr,
    int64_t* __restrict__ stats) {
  const int lane = threadIdx.x;
  // every load of the table goes out before the top-k: one memory round trip
  SlotRegs<PERC> t;
  t.load(stamp, slot_expert, cap);
  ExpertRegs<PER> table;
  table.load(slot_of, n_experts);
  StatsPrefetch prev;
  prev.load(stats);
  int64_t step_raw = *step_ptr;
  float lv[PER];
  load_logits<PER>(logits, n_experts, lv);
  // the step passes through this (empty) statement once every load above is
  // issued: the compiler would otherwise load it where the resolve needs it,
  // after the top-k, a second memory round trip
  asm volatile("" : "+s"(step_raw));
  const int64_t step = step_raw + 1;
  int32_t id;
  float wt;
  wave_topk_of<PER>(lv, n_experts, top_k, &id, &wt);
  if (lane < top_k) {
    ids[lane] = id;
    weights[lane] = wt;
  }
  // the picks are already one per lane: resolve them in pick order
  const int32_t my_e = lane < top_k ? id : -1;
  const int32_t found = table.lookup(my_e < 0 ? 0 : my_e);
  const int32_t my_s = my_e < 0 ? -1 : found;
  int32_t nm = 0;
  int64_t hits = 0;
  resolve_chunk<PERC>(t, my_e, my_s, top_k, 0, step, cap, slot_of, slot_expert, out_slot,
                      fetch_slot, fetch_expert, nm, hits);
  resolve_finish<PERC>(t, step, nm, hits, cap, stamp, step_ptr, nmiss_ptr, stats, prev);
}

// The decode step's route + fetch: the top-k and slot resolve of one token
// (topk_resolve_kernel's decisions) and the fetch of its misses (fetch.hip's
// pieces) in one launch, on the fetch's grid.  Every workgroup's first wave
// makes the same decisions from the same inputs (the logits and the current
// table, which no workgroup of this launch writes) and puts the miss list
// in LDS; workgroup 0 also writes the outputs and the next table.  The slot
// table is double-buffered: the call counted `step` (the logits launch before
// it adds one) reads buffer (step - 1) & 1 and writes buffer step & 1, so no
// workgroup can see a half-written table.  Saves the separate resolve launch
// and the fetch's reload of the miss list.
template <int PER, int PERC>
__global__ __launch_bounds__(kFetchThreads) void route_fetch_kernel(
    FetchArgs a, const float* __restrict__ logits, int32_t n_experts, int32_t top_k,
    int32_t* __restrict__ ids, float* __restrict__ weights, int32_t* __restrict__ slot_of,
    int32_t* __restrict__ slot_expert, int64_t* __restrict__ stamp, int32_t cap,
    const int64_t* __restrict__ step_ptr, int32_t* __restrict__ out_slot,
    int32_t* __restrict__ fetch_slot, int32_t* __restrict__ fetch_expert,
    int32_t* __restrict__ nmiss_ptr, int64_t* __restrict__ stats) {
  __shared__ u32x4 stage[16 * 33];
  __shared__ int32_t job_e[kMaxTopK], job_s[kMaxTopK], job_n;
  int32_t slot_r;
  bool miss_r;
  route_wave<PER, PERC>(logits, n_experts, top_k, ids, weights, slot_of, slot_expert, stamp, cap,
                        step_ptr, out_slot, fetch_slot, fetch_expert, nmiss_ptr, stats, job_e,
                        job_s, nullptr, &job_n, slot_r, miss_r);
  __syncthreads();
  const int64_t total = static_cast<int64_t>(job_n) * a.pieces_per_job;
  for (int64_t item = blockIdx.x; item < total; item += gridDim.x) {
    const int64_t j = item / a.pieces_per_job;
    // job_e/job_s are the same in every lane: made scalar, so the piece's
    // addressing stays scalar as in the fetch kernel
    fetch_piece(a, item - j * a.pieces_per_job, __builtin_amdgcn_readfirstlane(job_e[j]),
                __builtin_amdgcn_readfirstlane(job_s[j]), stage);
  }
}

int launch_decode_logits(const void* x, const void* w, const float* bias, int32_t hidden,
                         int32_t n_experts, int bf16_logits, float* logits, int64_t* step_inc,
                         hipStream_t s, int32_t* ticket) {
  hipLaunchKernelGGL(router_logits_kernel<1>, dim3((n_experts + kLogitWaves - 1) / kLogitWaves, 1),
                     dim3(64 * kLogitWaves), 0, s, static_cast<const uint16_t*>(x),
                     static_cast<const uint16_t*>(w), bias, 1, hidden, n_experts, bf16_logits,
                     logits, step_inc, ticket);
  return check_launch("router_logits_kernel");
}

int launch_router_logits(const void* x, const void* w, const float* bias, int32_t tokens,
                         int32_t hidden, int32_t n_experts, int bf16_logits, float* logits,
                         hipStream_t s) {
  const dim3 grid((n_experts + kLogitWaves - 1) / kLogitWaves,
                  (tokens + kTokBlock - 1) / kTokBlock);
  if (tokens >= kLogitMmaFrom && hidden % 32 == 0) {
    hipLaunchKernelGGL(router_logits_mma_kernel, dim3((n_experts + 15) / 16, (tokens + 15) / 16),
                       dim3(64 * kLogitMmaWaves), 0, s, static_cast<const uint16_t*>(x),
                       static_cast<const uint16_t*>(w), bias, tokens, hidden, n_experts,
                       bf16_logits, logits);
  } else if (tokens == 1)
    hipLaunchKernelGGL(router_logits_kernel<1>, grid, dim3(64 * kLogitWaves), 0, s,
                       static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), bias,
                       tokens, hidden, n_experts, bf16_logits, logits, nullptr, nullptr);
  else
    hipLaunchKernelGGL(router_logits_kernel<kTokBlock>, grid, dim3(64 * kLogitWaves), 0, s,
                       static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), bias,
                       tokens, hidden, n_experts, bf16_logits, logits, nullptr, nullptr);
  return check_launch("router_logits_kernel");
}

}  // namespace moe

using namespace moe;

extern "C" int moe_router_topk(const void* x, const void* w, const float* bias,
                               int32_t logit_dtype, int32_t tokens, int32_t hidden,
                               int32_t n_experts, int32_t top_k, float* logits, void* ids,
                               int32_t ids_dtype, void* weights, int32_t w_dtype, void* stream) {
  MOE_REQUIRE(tokens >= 0, "moe_router_topk: tokens < 0");
  MOE_REQUIRE(logit_dtype == MOE_F32 || logit_dtype == MOE_BF16,
              "moe_router_topk: logit_dtype must be MOE_F32 or MOE_BF16");
  MOE_REQUIRE(hidden > 0 && hidden % 8 == 0, "moe_router_topk: hidden %% 8 != 0 (%d)", hidden);
  MOE_REQUIRE(top_k >= 1 && top_k <= kMaxTopK && top_k <= n_experts && n_experts <= 4096,
              "moe_router_topk: need 1 <= top_k <= min(32, n_experts), n_experts <= 4096");
  MOE_REQUIRE(ids_dtype == MOE_I32 || ids_dtype == MOE_I64, "moe_router_topk: bad ids_dtype");
  MOE_REQUIRE(w_dtype == MOE_F32 || w_dtype == MOE_BF16, "moe_router_topk: bad w_dtype");
  if (tokens == 0) return MOE_OK;   // an empty call touches nothing (its tensors may be NULL)
  MOE_REQUIRE(x && w && logits && ids && weights, "moe_router_topk: NULL pointer");
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0,
              "moe_router_topk: x and w must be 16-byte aligned");
  const dim3 grid((n_experts + kLogitWaves - 1) / kLogitWaves,
                  (tokens + kTokBlock - 1) / kTokBlock);
  MOE_REQUIRE(grid.y <= 65535, "moe_router_topk: too many tokens (%d)", tokens);
  hipStream_t s = as_stream(stream);
  int rc = launch_router_logits(x, w, bias, tokens, hidden, n_experts,
                                logit_dtype == MOE_BF16 ? 1 : 0, logits, s);
  if (rc) return rc;
  const int i64 = ids_dtype == MOE_I64 ? 1 : 0, bf = w_dtype == MOE_BF16 ? 1 : 0;
  if (n_experts <= 256)
    hipLaunchKernelGGL(router_topk_kernel<4>, dim3(tokens), dim3(64), 0, s, logits, n_experts,
                       top_k, ids, i64, weights, bf);
  else if (n_experts <= 1024)
    hipLaunchKernelGGL(router_topk_kernel<16>, dim3(tokens), dim3(64), 0, s, logits, n_experts,
                       top_k, ids, i64, weights, bf);
  else
    hipLaunchKernelGGL(router_topk_kernel<64>, dim3(tokens), dim3(64), 0, s, logits, n_experts,
                       top_k, ids, i64, weights, bf);
  return check_launch("moe_router_topk(topk)");
}

extern "C" int moe_route_resolve(const void* x, const void* w, const float* bias,
                                 int32_t logit_dtype, int32_t hidden,
                                 int32_t n_experts, int32_t top_k, float* logits, int32_t* ids,
                                 float* weights, int32_t* slot_of, int32_t* slot_expert,
                                 int64_t* slot_stamp, int32_t cap, int64_t* step,
                                 int32_t* out_slot, int32_t* fetch_slot, int32_t* fetch_expert,
                                 int32_t* nmiss, int64_t* stats, void* stream) {
  MOE_REQUIRE(x && w && logits && ids && weights && slot_of && slot_expert && slot_stamp && step &&
                  out_slot && fetch_slot && fetch_expert && nmiss,
              "moe_route_resolve: NULL pointer");
  MOE_REQUIRE(logit_dtype == MOE_F32 || logit_dtype == MOE_BF16,
              "moe_route_resolve: logit_dtype must be MOE_F32 or MOE_BF16");
  MOE_REQUIRE(hidden > 0 && hidden % 8 == 0, "moe_route_resolve: hidden %% 8 != 0 (%d)", hidden);
  MOE_REQUIRE(top_k >= 1 && top_k <= kMaxTopK && top_k <= n_experts && n_experts <= 4096,
              "moe_route_resolve: need 1 <= top_k <= min(32, n_experts), n_experts <= 4096");
  MOE_REQUIRE(cap >= 1 && cap <= kMaxCap, "moe_route_resolve: need 1 <= cap <= %d", kMaxCap);
  // more ids than slots would hand one slot to two ids of this call
  MOE_REQUIRE(top_k <= cap, "moe_route_resolve: top_k (%d) exceeds the cache capacity (%d)",
              top_k, cap);
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0,
              "moe_route_resolve: x and w must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(router_logits_kernel<1>, dim3((n_experts + kLogitWaves - 1) / kLogitWaves, 1),
                     dim3(64 * kLogitWaves), 0, s,
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), bias, 1,
                     hidden, n_experts, logit_dtype == MOE_BF16 ? 1 : 0, logits, nullptr, nullptr);
  int rc = check_launch("moe_route_resolve(logits)");
  if (rc) return rc;
#define MOE_TR(PE, PC)                                                                          \
  hipLaunchKernelGGL((topk_resolve_kernel<PE, PC>), dim3(1), dim3(64), 0, s, logits, n_experts, \
                     top_k, ids, weights, slot_of, slot_expert, slot_stamp, cap, step, out_slot, \
                     fetch_slot, fetch_expert, nmiss, stats)
  if (n_experts <= 256) {
    if (cap <= 256) MOE_TR(4, 4); else if (cap <= 1024) MOE_TR(4, 16); else MOE_TR(4, 64);
  } else if (n_experts <= 1024) {
    if (cap <= 256) MOE_TR(16, 4); else if (cap <= 1024) MOE_TR(16, 16); else MOE_TR(16, 64);
  } else {
    if (cap <= 256) MOE_TR(64, 4); else if (cap <= 1024) MOE_TR(64, 16); else MOE_TR(64, 64);
  }
#undef MOE_TR
  return check_launch("moe_route_resolve(topk+resolve)");
}

extern "C" int moe_route_fetch(const void* x, const void* w, const float* bias, int32_t logit_dtype,
                               int32_t hidden, int32_t n_experts, int32_t top_k, float* logits,
                               int32_t* ids, float* weights, int32_t* slot_of,
                               int32_t* slot_expert, int64_t* slot_stamp, int32_t cap,
                               int64_t* step, int32_t* out_slot, int32_t* fetch_slot,
                               int32_t* fetch_expert, int32_t* nmiss, int64_t* stats,
                               const moe_fetch_pair* pairs, int32_t npairs,
                               int32_t blocks_per_job, void* stream) {
  MOE_REQUIRE(x && w && logits && ids && weights && slot_of && slot_expert && slot_stamp && step &&
                  out_slot && fetch_slot && fetch_expert && nmiss,
              "moe_route_fetch: NULL pointer");
  MOE_REQUIRE(logit_dtype == MOE_F32 || logit_dtype == MOE_BF16,
              "moe_route_fetch: logit_dtype must be MOE_F32 or MOE_BF16");
  MOE_REQUIRE(hidden > 0 && hidden % 8 == 0, "moe_route_fetch: hidden %% 8 != 0 (%d)", hidden);
  MOE_REQUIRE(top_k >= 1 && top_k <= kMaxTopK && top_k <= n_experts && n_experts <= 1024,
              "moe_route_fetch: need 1 <= top_k <= min(32, n_experts), n_experts <= 1024");
  MOE_REQUIRE(cap >= 1 && cap <= 1024, "moe_route_fetch: need 1 <= cap <= 1024");
  MOE_REQUIRE(top_k <= cap, "moe_route_fetch: top_k (%d) exceeds the cache capacity (%d)",
              top_k, cap);
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0,
              "moe_route_fetch: x and w must be 16-byte aligned");
  MOE_REQUIRE(blocks_per_job >= 1 && blocks_per_job <= 4096,
              "moe_route_fetch: need 1 <= blocks_per_job <= 4096");
  FetchArgs a;
  const int rc0 = fetch_args(pairs, npairs, top_k, &a);
  if (rc0 != MOE_OK) return rc0;
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(router_logits_kernel<1>, dim3((n_experts + kLogitWaves - 1) / kLogitWaves, 1),
                     dim3(64 * kLogitWaves), 0, s,
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), bias, 1,
                     hidden, n_experts, logit_dtype == MOE_BF16 ? 1 : 0, logits, step, nullptr);
  int rc = check_launch("moe_route_fetch(logits)");
  if (rc) return rc;
  const int grid = blocks_per_job * (top_k < kFetchMaxJobsInGrid ? top_k : kFetchMaxJobsInGrid);
#define MOE_RF(PE, PC)                                                                          \
  hipLaunchKernelGGL((route_fetch_kernel<PE, PC>), dim3(grid), dim3(kFetchThreads), 0, s, a,    \
                     logits, n_experts, top_k, ids, weights, slot_of, slot_expert, slot_stamp,   \
                     cap, step, out_slot, fetch_slot, fetch_expert, nmiss, stats)
  if (n_experts <= 256) {
    if (cap <= 256) MOE_RF(4, 4); else MOE_RF(4, 16);
  } else {
    if (cap <= 256) MOE_RF(16, 4); else MOE_RF(16, 16);
  }
#undef MOE_RF
  return check_launch("moe_route_fetch(route+fetch)");
}
