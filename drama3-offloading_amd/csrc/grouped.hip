// Grouped W8A8 expert FFN for many tokens (prefill, batched decode): token
// rows are permuted into per-expert segments (permute.hip), every expert's
// weights are read from HBM once for all of its tokens, and the results are
// un-permuted with the routing weights.
//
//   quant_rows:  x [T, H] bf16 -> xq [T, H] e4m3, xs [T, H/128]   (per token)
//   gateup:      grid (E, I/128), 4 waves.  Workgroup = expert e, quant
//                group jb of the intermediate: wave w owns gate columns
//                j in [jb*128 + 32w, +32) and the up columns j + I, i.e. four
//                16-column MFMA tiles, for up to 64 tokens of the segment at a
//                time.  After the 2048-deep reduction it forms
//                a = SiLU(gate) * up, takes the per-token amax over the group's
//                128 columns across the four waves, and writes aq/as rows in
//                permuted order.
//   down:        grid (E, H/256), 4 waves x 4 tiles of 16 output features;
//                the activations are the expert's contiguous aq rows.  y rows
//                in permuted order, float32.
//   unpermute:   out[t] = sum_k w[t,k] * y[pos[t,k]] (permute.hip).
//
// MFMA 16x16x128 e4m3 with the same operand roles as the decode GEMV:
// weight rows are the A operand, activations the B operand (here one token
// per B column), every lane supplies the same 32-byte reduction slice, block
// scales multiply each 128-deep block result as weight_scale *
// activation_scale, and the blocks are summed in the same order -- so every
// (token, expert) row computed here is bit-identical to the decode GEMV's.
#include "common.hpp"
#include "grouped.hpp"

namespace moe {

constexpr int kMTiles = 4;           // token tiles of 16 held at once (64 tokens)

// --------------------------------------------------------------- quant x

__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t* __restrict__ x,
                                                         int32_t hidden, uint8_t* __restrict__ xq,
                                                         float* __restrict__ xs) {
  // one workgroup per token; 16 threads x 8 values per 128-group
  const int64_t t = blockIdx.x;
  const uint16_t* xr = x + t * hidden;
  for (int base = 0; base < hidden; base += 2048) {
    const int i = base + threadIdx.x * 8;
    float v[8];
    float amax = 0.0f;
    if (i < hidden) {
      const uint4 raw = *reinterpret_cast<const uint4*>(xr + i);
      const uint32_t r[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = __uint_as_float(r[j] << 16);
        v[2 * j + 1] = __uint_as_float(r[j] & 0xffff0000u);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    if (i < hidden) {
      const float s = act_scale(amax);
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) lo |= quant_e4m3(v[j], s) << (8 * j);
#pragma unroll
      for (int j = 0; j < 4; ++j) hi |= quant_e4m3(v[4 + j], s) << (8 * j);
      *reinterpret_cast<uint2*>(xq + t * hidden + i) = make_uint2(lo, hi);
      if ((threadIdx.x & 15) == 0) xs[t * (hidden >> 7) + (i >> 7)] = s;
    }
  }
}

// --------------------------------------------------------------- gate/up

// Weight rows are the A operand (16 rows per tile, as in the decode GEMV) and
// the tokens the B operand (16 token columns per tile): lane l's result
// element i is weight row 4*(l/16) + i of the tile for token column l % 16.
__global__ __launch_bounds__(256) void grouped_gateup_kernel(
    const uint8_t* __restrict__ xq, const float* __restrict__ xs,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_pairs, int32_t top_k, const uint8_t* __restrict__ w13,
    const float* __restrict__ s13, int64_t w13_es, int64_t s13_es, int32_t hidden, int32_t inter,
    uint8_t* __restrict__ aq, float* __restrict__ as_) {
  __shared__ int32_t tok[kMTiles * 16];
  __shared__ float colmax[4][kMTiles * 16];
  const int e = blockIdx.x;
  const int jb = blockIdx.y;
  const int32_t m_e = counts[e];
  if (m_e == 0) return;
  const int32_t off = offsets[e];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4;
  const int col = lane & 15;
  const int G = hidden >> 7;
  const int Gi = inter >> 7;
  // the four row tiles of this wave: gate j0, gate j0+16, up j0, up j0+16
  const int j0 = jb * 128 + wave * 32;
  int rows[4];
  rows[0] = j0;
  rows[1] = j0 + 16;
  rows[2] = inter + j0;
  rows[3] = inter + j0 + 16;
  const uint8_t* wb = w13 + static_cast<int64_t>(e) * w13_es;
  const float* sb = s13 + static_cast<int64_t>(e) * s13_es;
  for (int m0 = 0; m0 < m_e; m0 += kMTiles * 16) {
    const int mcols = min(kMTiles * 16, m_e - m0);
    const int ntiles = (mcols + 15) >> 4;
    __syncthreads();
    if (threadIdx.x < kMTiles * 16)
      tok[threadIdx.x] = threadIdx.x < mcols ? sorted_pairs[off + m0 + threadIdx.x] / top_k : -1;
    __syncthreads();
    v4f acc[kMTiles][4];
#pragma unroll
    for (int mt = 0; mt < kMTiles; ++mt)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[mt][t] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int g = 0; g < G; ++g) {
      v8i wa[4];
      float ws[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        wa[t] = load_op32_nt(wb + static_cast<int64_t>(rows[t] + col) * hidden + g * 128 + q * 32);
        ws[t] = sb[(rows[t] >> 7) * G + g];
      }
#pragma unroll
      for (int mt = 0; mt < kMTiles; ++mt) {
        if (mt < ntiles) {
          const int tc = tok[mt * 16 + col];
          v8i xb = v8i{0, 0, 0, 0, 0, 0, 0, 0};
          float xsc = 0.0f;
          if (tc >= 0) {
            xb = load_op32(xq + static_cast<int64_t>(tc) * hidden + g * 128 + q * 32);
            xsc = xs[static_cast<int64_t>(tc) * G + g];
          }
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const v4f z = {0.f, 0.f, 0.f, 0.f};
            const v4f d = mfma_e4m3_16x16x128(wa[t], xb, z);
            const float sc = ws[t] * xsc;
            block_fma(acc[mt][t], d, sc);
          }
        }
      }
    }
    // a = SiLU(gate) * up for j = j0 + 16t + 4q + i; per-token amax over the
    // 128 columns of group jb (8 per lane, 4 row groups, 4 waves)
    float av[kMTiles][2][4];
#pragma unroll
    for (int mt = 0; mt < kMTiles; ++mt) {
      float mx = 0.0f;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          av[mt][t][i] = silu_mul(acc[mt][t][i], acc[mt][t + 2][i]);
          mx = fmaxf(mx, fabsf(av[mt][t][i]));
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      if (q == 0) colmax[wave][mt * 16 + col] = mx;
    }
    __syncthreads();
#pragma unroll
    for (int mt = 0; mt < kMTiles; ++mt) {
      const int c = mt * 16 + col;
      if (mt < ntiles && c < mcols) {
        const float amax = fmaxf(fmaxf(colmax[0][c], colmax[1][c]), fmaxf(colmax[2][c], colmax[3][c]));
        const float sc = act_scale(amax);
        const int64_t pos = off + m0 + c;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          uint32_t wd = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) wd |= quant_e4m3(av[mt][t][i], sc) << (8 * i);
          *reinterpret_cast<uint32_t*>(aq + pos * inter + j0 + t * 16 + 4 * q) = wd;
        }
        if (wave == 0 && q == 0) as_[pos * Gi + jb] = sc;
      }
    }
  }
}

// --------------------------------------------------------------- down

// w2 rows (output features) are the A operand, the expert's contiguous aq
// rows (tokens) the B operand; lane l's element i is feature 4*(l/16) + i of
// the tile for token column l % 16.
__global__ __launch_bounds__(256) void grouped_down_kernel(
    const uint8_t* __restrict__ aq, const float* __restrict__ as_,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const uint8_t* __restrict__ w2, const float* __restrict__ s2, int64_t w2_es, int64_t s2_es,
    int32_t hidden, int32_t inter, float* __restrict__ y) {
  const int e = blockIdx.x;
  const int32_t m_e = counts[e];
  if (m_e == 0) return;
  const int32_t off = offsets[e];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4;
  const int col = lane & 15;
  const int Gi = inter >> 7;
  const int c0 = blockIdx.y * 256 + wave * 64;
  const uint8_t* wb = w2 + static_cast<int64_t>(e) * w2_es;
  const float* sb = s2 + static_cast<int64_t>(e) * s2_es;
  for (int m0 = 0; m0 < m_e; m0 += kMTiles * 16) {
    const int mcols = min(kMTiles * 16, m_e - m0);
    const int ntiles = (mcols + 15) >> 4;
    v4f acc[kMTiles][4];
#pragma unroll
    for (int mt = 0; mt < kMTiles; ++mt)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[mt][t] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int g = 0; g < Gi; ++g) {
      v8i wa[4];
      float ws[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int c = c0 + t * 16;
        wa[t] = load_op32_nt(wb + static_cast<int64_t>(c + col) * inter + g * 128 + q * 32);
        ws[t] = sb[(c >> 7) * Gi + g];
      }
#pragma unroll
      for (int mt = 0; mt < kMTiles; ++mt) {
        if (mt < ntiles) {
          const int cc = mt * 16 + col;
          v8i ab = v8i{0, 0, 0, 0, 0, 0, 0, 0};
          float asc = 0.0f;
          if (cc < mcols) {
            const int64_t pos = off + m0 + cc;
            ab = load_op32(aq + pos * inter + g * 128 + q * 32);
            asc = as_[pos * Gi + g];
          }
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const v4f z = {0.f, 0.f, 0.f, 0.f};
            const v4f d = mfma_e4m3_16x16x128(wa[t], ab, z);
            const float sc = ws[t] * asc;
            block_fma(acc[mt][t], d, sc);
          }
        }
      }
    }
#pragma unroll
    for (int mt = 0; mt < kMTiles; ++mt) {
      const int cc = mt * 16 + col;
      if (mt < ntiles && cc < mcols) {
        float* yr = y + static_cast<int64_t>(off + m0 + cc) * hidden + c0 + 4 * q;
#pragma unroll
        for (int t = 0; t < 4; ++t)
          *reinterpret_cast<float4*>(yr + t * 16) =
              make_float4(acc[mt][t][0], acc[mt][t][1], acc[mt][t][2], acc[mt][t][3]);
      }
    }
  }
}

// --------------------------------------------------------------- driver

GroupedLayout grouped_layout(int32_t tokens, int32_t top_k, int32_t n_experts, int32_t hidden,
                             int32_t inter) {
  GroupedLayout L;
  const int64_t P = static_cast<int64_t>(tokens) * top_k;
  auto align = [](size_t v) { return (v + 255) & ~static_cast<size_t>(255); };
  size_t o = 0;
  L.counts = o;       o = align(o + sizeof(int32_t) * n_experts);
  L.offsets = o;      o = align(o + sizeof(int32_t) * (n_experts + 1));
  L.sorted = o;       o = align(o + sizeof(int32_t) * P);
  L.pos = o;          o = align(o + sizeof(int32_t) * P);
  L.xq = o;           o = align(o + static_cast<size_t>(tokens) * hidden);
  L.xs = o;           o = align(o + sizeof(float) * tokens * (hidden / 128));
  L.aq = o;           o = align(o + static_cast<size_t>(P) * inter);
  L.as = o;           o = align(o + sizeof(float) * P * (inter / 128));
  L.y = o;            o = align(o + sizeof(float) * P * hidden);
  L.total = o;
  return L;
}

int launch_grouped(const uint16_t* x, const void* ids, int ids64, const void* weights, int wbf16,
                   int32_t tokens, int32_t top_k, const uint8_t* w13, const float* s13,
                   const uint8_t* w2, const float* s2, const moe_expert_strides& es,
                   int32_t n_experts, int32_t hidden, int32_t inter, const uint16_t* residual,
                   uint16_t* out, char* ws, hipStream_t s) {
  const GroupedLayout L = grouped_layout(tokens, top_k, n_experts, hidden, inter);
  int32_t* counts = reinterpret_cast<int32_t*>(ws + L.counts);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + L.offsets);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + L.sorted);
  int32_t* pos = reinterpret_cast<int32_t*>(ws + L.pos);
  uint8_t* xq = reinterpret_cast<uint8_t*>(ws + L.xq);
  float* xs = reinterpret_cast<float*>(ws + L.xs);
  uint8_t* aq = reinterpret_cast<uint8_t*>(ws + L.aq);
  float* as_ = reinterpret_cast<float*>(ws + L.as);
  float* y = reinterpret_cast<float*>(ws + L.y);
  const int64_t P = static_cast<int64_t>(tokens) * top_k;
  int rc = launch_permute(ids, ids64, P, n_experts, counts, offsets, sorted, pos, s);
  if (rc) return rc;
  hipLaunchKernelGGL(quant_rows_kernel, dim3(tokens), dim3(256), 0, s, x, hidden, xq, xs);
  rc = check_launch("moe_fp8_moe_forward(quant)");
  if (rc) return rc;
  hipLaunchKernelGGL(grouped_gateup_kernel, dim3(n_experts, inter / 128), dim3(256), 0, s, xq, xs,
                     counts, offsets, sorted, top_k, w13, s13, es.w13, es.s13, hidden, inter, aq,
                     as_);
  rc = check_launch("moe_fp8_moe_forward(grouped gate/up)");
  if (rc) return rc;
  hipLaunchKernelGGL(grouped_down_kernel, dim3(n_experts, hidden / 256), dim3(256), 0, s, aq, as_,
                     counts, offsets, w2, s2, es.w2, es.s2, hidden, inter, y);
  rc = check_launch("moe_fp8_moe_forward(grouped down)");
  if (rc) return rc;
  return launch_unpermute(y, pos, weights, wbf16, tokens, top_k, hidden, residual, out, s);
}

}  // namespace moe
