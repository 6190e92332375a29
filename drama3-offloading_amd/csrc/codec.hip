// Entropy-coded expert records: fewer bytes over the host link, decoded on
// the GPU into byte-exact cache slots.
//
// The fp8 (e4m3) weights of a record are 1 sign, 4 exponent and 3 mantissa
// bits.  Block-scaled weights use few exponents (the 128x128 block maximum
// maps to 448), so the exponent nibble carries about 2.6 bits; sign and
// mantissa are close to uniform.  A record's fp8 bytes are cut into blocks
// of 8192 and each block is stored as
//
//   [0, 4096)        nibble plane: nibble byte m of lane l (symbols
//                    x[128l + 2m], x[128l + 2m + 1]) = nib(first) |
//                    nib(second) << 4, nib(v) = (sign << 3) | mantissa, at
//                    16 * (64 * (m / 16) + l) + m % 16 -- each wave-wide
//                    16-byte load then reads 1 KiB contiguous
//   [4096, 4160)     lane header: byte l = length in bytes of stream l
//   [4160, ...)      64 streams, stream l the exponents of x[128l, 128l+128)
//                    as canonical Huffman codes (at most 6 bits), written
//                    least significant bit first, each stream byte-padded
//   padded to 16 bytes.
//
// The bytes after the fp8 part (the block scales) follow raw.  Records are
// 256-byte aligned in the coded pool; where each record and each of its
// blocks starts is a device-resident index, so the fetch kernel needs no
// host read to find them.
//
// Decoding: one wave per block.  The header and streams go to LDS, the
// nibble plane straight to registers (lane l takes its 64 bytes); each
// lane finds its stream's start with a wave prefix sum of the header, then
// decodes its 128 exponents two at a time with a 4096-entry table in LDS (12
// peeked bits always hold two whole codes: entry = both symbols and their
// total length) and writes its 128 bytes to the cache slot.  The next stream
// word is read one step ahead, so a step waits on one LDS access.
//
// Two launches use the decoder: moe_fetch_coded (the miss list read from
// device memory) and moe_route_fetch_coded (the decode step's route made by
// every workgroup first, the miss list then read from LDS).
#include <string.h>

#include <algorithm>
#include <atomic>
#include <system_error>
#include <thread>
#include <vector>

#include "common.hpp"
#include "route.hpp"

namespace moe {

constexpr int kCodecBlock = 8192;                 // fp8 bytes per block
constexpr int kCodecLanes = 64;
constexpr int kCodecPerLane = kCodecBlock / kCodecLanes;   // 128 symbols
constexpr int kCodecPlane = kCodecBlock / 2;      // nibble plane bytes
constexpr int kCodecHeader = kCodecLanes;         // one length byte per lane
constexpr int kCodecMaxLen = 6;                   // longest code, bits (two codes fit 12)
constexpr int kCodecPeek = 2 * kCodecMaxLen;      // bits one table entry decodes
constexpr int kCodecLutSize = 1 << kCodecPeek;    // 4096 entries of two symbols
constexpr int kCodecAlign = 16;                   // block size granule
constexpr int kCodecMaxBlock = kCodecPlane + kCodecHeader + kCodecBlock + kCodecAlign;

// -------------------------------------------------------------- device

constexpr int kCodecWaves = 4;                    // waves per workgroup, one block each
constexpr int kCodecLds = kCodecHeader + kCodecBlock + 64;   // header + streams + over-read

__device__ __forceinline__ int wave_exclusive_sum(int v) {
  const int lane = threadIdx.x & 63;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int n = __shfl_up(incl, o, 64);
    if (lane >= o) incl += n;
  }
  return incl - v;
}

// Where unit u (job u / nblk, block u % nblk) comes from and goes to; the
// miss list through `jobs` (expert(j), slot(j), both uniform).
struct CodedUnit {
  const uint8_t* src;   // coded block (host)
  uint8_t* dst;         // decoded block (cache slot)
  int rest;             // bytes after the nibble plane: header + streams, multiple of 16
};

template <class Jobs>
__device__ __forceinline__ CodedUnit coded_unit(int64_t u, int32_t nblk, const uint8_t* pool,
                                                const int64_t* rec_off, const uint32_t* blk_off,
                                                const Jobs& jobs, uint8_t* cache,
                                                int64_t slot_bytes) {
  const int64_t j = u / nblk;
  const int b = static_cast<int>(u - j * nblk);
  const int64_t e = jobs.expert(j);
  const uint32_t* bo = blk_off + e * (static_cast<int64_t>(nblk) + 1);
  CodedUnit c;
  c.src = pool + rec_off[e] + bo[b];
  c.dst = cache + jobs.slot(j) * slot_bytes + static_cast<int64_t>(b) * kCodecBlock;
  c.rest = static_cast<int>(bo[b + 1] - bo[b]) - kCodecPlane;
  return c;
}

// The miss list in device memory (moe_fetch_coded: the resolve's outputs).
struct JobsInMemory {
  const int32_t* fexp;
  const int32_t* fslot;
  __device__ __forceinline__ int64_t expert(int64_t j) const { return fexp[j]; }
  __device__ __forceinline__ int64_t slot(int64_t j) const { return fslot[j]; }
};

// The miss list in LDS (the route made by the same launch), made scalar.
struct JobsInLds {
  const int32_t* je;
  const int32_t* js;
  __device__ __forceinline__ int64_t expert(int64_t j) const {
    return __builtin_amdgcn_readfirstlane(je[j]);
  }
  __device__ __forceinline__ int64_t slot(int64_t j) const {
    return __builtin_amdgcn_readfirstlane(js[j]);
  }
};

// The host loads of one coded block for this lane: its 64 nibble-plane bytes
// and its share of header + streams.  Only the wave-wide loads that reach
// into the block are issued (a uniform branch on the block's size); in the
// last of them, lanes past the block re-read its last piece, a line that
// the same instruction reads anyway.
constexpr int kCodecRestLoads = (kCodecHeader + kCodecPerLane * kCodecMaxLen / 8 * kCodecLanes +
                                 1023) / 1024;   // 7 for 6-bit codes

struct CodedLoads {
  u32x4 nib[4];
  u32x4 rest[kCodecRestLoads];
  __device__ __forceinline__ void issue(const CodedUnit& c, int lane) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      nib[k] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(c.src) + kCodecLanes * k + lane);
#pragma unroll
    for (int k = 0; k < kCodecRestLoads; ++k) {
      if (k * 1024 >= c.rest) break;              // c.rest is wave-uniform
      const int i = min(k * 1024 + lane * 16, c.rest - 16);
      rest[k] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(c.src + kCodecPlane + i));
    }
  }
};

// The fetch of nm coded records by the grid's waves: job j copies coded
// record jobs.expert(j) into cache slot jobs.slot(j), decoded.  The nm * nblk
// blocks are dealt to the waves round-robin; a wave loads a block, then
// decodes it.  Waves are spread thin (4 per workgroup, one workgroup per CU
// at the default grid), and at any time only the waves between blocks have
// host reads outstanding.  Measured on MI355X, 8 records per launch: 389 us
// against 447 us for the raw fetch; issuing the next block's loads before
// decoding the current one (every wave holding ~7 KB in flight) lowered the
// link's rate from ~56 to ~52 GB/s and took 412 us.  The raw tails (block
// scales) are copied first, one per wave.  `lut` is the decode table in LDS.
template <class Jobs>
__device__ __forceinline__ void coded_fetch_run(
    const Jobs& jobs, int32_t nm, const uint8_t* __restrict__ pool,
    const int64_t* __restrict__ rec_off, const uint32_t* __restrict__ blk_off, int32_t nblk,
    int64_t tail, const uint16_t* lut, uint8_t* __restrict__ cache, int64_t slot_bytes,
    uint8_t (*lds)[kCodecLds]) {
  // wave-uniform as a scalar: block indices and addresses then come from
  // scalar loads, which do not wait behind this wave's host loads
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t gw = static_cast<int64_t>(blockIdx.x) * kCodecWaves + wave;   // global wave
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kCodecWaves;
  for (int64_t j = gw; j < nm; j += nwaves) {     // raw tails
    const int64_t e = jobs.expert(j);
    const uint8_t* src = pool + rec_off[e] + blk_off[e * (static_cast<int64_t>(nblk) + 1) + nblk];
    uint8_t* dst = cache + jobs.slot(j) * slot_bytes + static_cast<int64_t>(nblk) * kCodecBlock;
    for (int64_t i = lane * 16; i < tail; i += 64 * 16)
      *reinterpret_cast<u32x4*>(dst + i) = *reinterpret_cast<const u32x4*>(src + i);
  }
  const int64_t units = static_cast<int64_t>(nm) * nblk;
  if (gw >= units) return;                        // this wave has no block (no barrier follows)
  const uint32_t* w32 = reinterpret_cast<const uint32_t*>(lds[wave]);
  CodedLoads ld;
  for (int64_t u = gw; u < units; u += nwaves) {
    const CodedUnit cur = coded_unit(u, nblk, pool, rec_off, blk_off, jobs, cache, slot_bytes);
    ld.issue(cur, lane);
    // this block's header + streams to LDS, its nibbles to registers
#pragma unroll
    for (int k = 0; k < kCodecRestLoads; ++k) {
      const int i = k * 1024 + lane * 16;
      if (i < cur.rest) *reinterpret_cast<u32x4*>(&lds[wave][i]) = ld.rest[k];
    }
    const uint32_t nw[16] = {ld.nib[0].x, ld.nib[0].y, ld.nib[0].z, ld.nib[0].w,
                             ld.nib[1].x, ld.nib[1].y, ld.nib[1].z, ld.nib[1].w,
                             ld.nib[2].x, ld.nib[2].y, ld.nib[2].z, ld.nib[2].w,
                             ld.nib[3].x, ld.nib[3].y, ld.nib[3].z, ld.nib[3].w};
    uint8_t* const dst = cur.dst;
    const int start = kCodecHeader + wave_exclusive_sum(lds[wave][lane]);
    // LSB-first bit reader: buf holds nbits >= 32 valid bits at every step
    // start; the word after them (nextw) is already read
    int wi = start >> 2;
    uint64_t buf = (static_cast<uint64_t>(w32[wi + 1]) << 32 | w32[wi]) >> ((start & 3) * 8);
    int nbits = 64 - (start & 3) * 8;
    wi += 2;
    uint32_t nextw = w32[wi];
    u32x4* d = reinterpret_cast<u32x4*>(dst + kCodecPerLane * lane);
#pragma unroll
    for (int q = 0; q < 8; ++q) {                 // 16 output bytes per q
      uint32_t ow[4];
#pragma unroll
      for (int h = 0; h < 8; ++h) {               // two symbols per step
        const int i = q * 16 + h * 2;             // first symbol of the step
        const uint32_t ent = lut[buf & (kCodecLutSize - 1)];
        const uint32_t len = ent >> 8;
        buf >>= len;
        nbits -= static_cast<int>(len);
        const bool take = nbits < 32;             // keep >= 32 bits for the next step
        buf |= take ? static_cast<uint64_t>(nextw) << nbits : 0ull;
        nbits += take ? 32 : 0;
        wi += take ? 1 : 0;
        nextw = w32[wi];
        const uint32_t nb = nw[i >> 3] >> ((i & 7) * 4);   // the step's two nibbles
        const uint32_t b0 = ((nb & 8) << 4) | ((ent & 15) << 3) | (nb & 7);
        const uint32_t b1 = (nb & 0x80) | (((ent >> 4) & 15) << 3) | ((nb >> 4) & 7);
        const uint32_t two = b0 | (b1 << 8);
        if ((h & 1) == 0)
          ow[h >> 1] = two;
        else
          ow[h >> 1] |= two << 16;
      }
      d[q] = u32x4{ow[0], ow[1], ow[2], ow[3]};
    }
  }
}

// Fetch of coded records: job j copies coded record fetch_expert[j] of the
// pool into cache slot fetch_slot[j], decoded; j < *nmiss (read on the
// device).
__global__ __launch_bounds__(64 * kCodecWaves) void fetch_coded_kernel(
    const uint8_t* __restrict__ pool, const int64_t* __restrict__ rec_off,
    const uint32_t* __restrict__ blk_off, int32_t nblk, int64_t tail,
    const uint16_t* __restrict__ lut_g, const int32_t* __restrict__ fexp,
    const int32_t* __restrict__ fslot, const int32_t* __restrict__ nmiss, int32_t max_jobs,
    uint8_t* __restrict__ cache, int64_t slot_bytes) {
  __shared__ __align__(16) uint8_t lds[kCodecWaves][kCodecLds];
  __shared__ uint16_t lut[kCodecLutSize];
  for (int i = threadIdx.x; i < kCodecLutSize; i += 64 * kCodecWaves) lut[i] = lut_g[i];
  __syncthreads();
  const int32_t nm = min(*nmiss, max_jobs);
  coded_fetch_run(JobsInMemory{fexp, fslot}, nm, pool, rec_off, blk_off, nblk, tail, lut, cache,
                  slot_bytes, lds);
}

// The decode step's route and the coded fetch of its misses in one launch
// (moe_route_fetch_coded): every workgroup's first wave makes the route
// (route.hpp: top-k + slot resolve on the double-buffered table, workgroup
// 0 writing the outputs and the next table) while the others copy the
// decode table to LDS; then all its waves decode the misses' blocks from
// the miss list in LDS, as fetch_coded_kernel does from memory.
template <int PER, int PERC>
__global__ __launch_bounds__(64 * kCodecWaves) void route_fetch_coded_kernel(
    const float* __restrict__ logits, int32_t n_experts, int32_t top_k, int32_t* __restrict__ ids,
    float* __restrict__ weights, int32_t* __restrict__ slot_of, int32_t* __restrict__ slot_expert,
    int64_t* __restrict__ stamp, int32_t cap, const int64_t* __restrict__ step_ptr,
    int32_t* __restrict__ out_slot, int32_t* __restrict__ fetch_slot,
    int32_t* __restrict__ fetch_expert, int32_t* __restrict__ nmiss_ptr,
    int64_t* __restrict__ stats, const uint8_t* __restrict__ pool,
    const int64_t* __restrict__ rec_off, const uint32_t* __restrict__ blk_off, int32_t nblk,
    int64_t tail, const uint16_t* __restrict__ lut_g, uint8_t* __restrict__ cache,
    int64_t slot_bytes) {
  __shared__ __align__(16) uint8_t lds[kCodecWaves][kCodecLds];
  __shared__ uint16_t lut[kCodecLutSize];
  __shared__ int32_t job_e[kMaxTopK], job_s[kMaxTopK], job_n;
  int32_t slot_r;
  bool miss_r;
  route_wave<PER, PERC>(logits, n_experts, top_k, ids, weights, slot_of, slot_expert, stamp, cap,
                        step_ptr, out_slot, fetch_slot, fetch_expert, nmiss_ptr, stats, job_e,
                        job_s, nullptr, &job_n, slot_r, miss_r);
  if (threadIdx.x >= 64)
    for (int i = threadIdx.x - 64; i < kCodecLutSize; i += 64 * (kCodecWaves - 1))
      lut[i] = lut_g[i];
  __syncthreads();
  const int32_t nm = __builtin_amdgcn_readfirstlane(job_n);
  coded_fetch_run(JobsInLds{job_e, job_s}, nm, pool, rec_off, blk_off, nblk, tail, lut, cache,
                  slot_bytes, lds);
}

// ---------------------------------------------------------------- host

struct CodeTable {
  uint8_t len[16];
  uint16_t rev[16];   // code bits reversed (LSB-first stream order)
};

// Canonical codes from lengths (0 = unused symbol); false if the lengths do
// not form a prefix code within kCodecMaxLen bits.
static bool make_codes(const uint8_t* len, CodeTable* t) {
  uint32_t kraft = 0;   // in units of 2^-kCodecMaxLen
  for (int s = 0; s < 16; ++s) {
    if (len[s] > kCodecMaxLen) return false;
    if (len[s]) kraft += 1u << (kCodecMaxLen - len[s]);
    t->len[s] = len[s];
  }
  if (kraft > (1u << kCodecMaxLen)) return false;
  uint32_t code = 0;
  int prev = 0;
  for (int l = 1; l <= kCodecMaxLen; ++l) {
    for (int s = 0; s < 16; ++s) {
      if (len[s] != l) continue;
      code <<= (l - prev);
      prev = l;
      uint32_t r = 0;
      for (int b = 0; b < l; ++b) r |= ((code >> b) & 1u) << (l - 1 - b);
      t->rev[s] = static_cast<uint16_t>(r);
      ++code;
    }
  }
  return true;
}

static inline uint8_t nib_of(uint8_t x) { return static_cast<uint8_t>(((x >> 4) & 8) | (x & 7)); }

// One block: returns its coded size (16-byte aligned), or -1 if a symbol
// has no code.
static int64_t encode_block(const uint8_t* x, const CodeTable& t, uint8_t* out) {
  for (int l = 0; l < kCodecLanes; ++l)
    for (int m = 0; m < kCodecPerLane / 2; ++m) {
      const uint8_t* v = x + l * kCodecPerLane + 2 * m;
      out[16 * (kCodecLanes * (m / 16) + l) + m % 16] =
          static_cast<uint8_t>(nib_of(v[0]) | (nib_of(v[1]) << 4));
    }
  uint8_t* hdr = out + kCodecPlane;
  uint8_t* st = hdr + kCodecHeader;
  int64_t pos = 0;
  for (int l = 0; l < kCodecLanes; ++l) {
    uint64_t acc = 0;
    int nb = 0;
    int64_t start = pos;
    for (int i = 0; i < kCodecPerLane; ++i) {
      const int s = (x[l * kCodecPerLane + i] >> 3) & 15;
      if (!t.len[s]) return -1;
      acc |= static_cast<uint64_t>(t.rev[s]) << nb;
      nb += t.len[s];
      while (nb >= 8) {
        st[pos++] = static_cast<uint8_t>(acc);
        acc >>= 8;
        nb -= 8;
      }
    }
    if (nb) st[pos++] = static_cast<uint8_t>(acc);
    hdr[l] = static_cast<uint8_t>(pos - start);    // <= 128
  }
  int64_t n = kCodecPlane + kCodecHeader + pos;
  while (n % kCodecAlign) out[n++] = 0;
  return n;
}

}  // namespace moe

using namespace moe;

// fn(i) for i < n, each on its own thread; an index whose thread cannot be
// started runs on the calling thread, so every started thread is joined.
template <class F>
static void run_threads(int n, const F& fn) {
  std::vector<std::thread> pool;
  pool.reserve(n);
  int i = 0;
  try {
    for (; i < n; ++i) pool.emplace_back(fn, i);
  } catch (const std::system_error&) {
    for (; i < n; ++i) fn(i);
  }
  for (auto& th : pool) th.join();
}

// The host entry points below run worker threads; an allocation failure is
// reported as MOE_EINVAL, never thrown across the C ABI.
extern "C" int moe_codec_histogram(const void* records, int64_t n_records, int64_t record_bytes,
                                   int64_t fp8_bytes, uint64_t* hist, int32_t threads) try {
  MOE_REQUIRE(records && hist, "moe_codec_histogram: NULL pointer");
  MOE_REQUIRE(n_records >= 0 && fp8_bytes >= 0 && fp8_bytes <= record_bytes,
              "moe_codec_histogram: bad sizes");
  const int nt = std::max(1, std::min<int>(threads, 64));
  std::vector<std::vector<uint64_t>> part(nt, std::vector<uint64_t>(16, 0));
  run_threads(nt, [&](int w) {
    for (int64_t r = w; r < n_records; r += nt) {
      const uint8_t* x = static_cast<const uint8_t*>(records) + r * record_bytes;
      uint64_t h[16] = {0};
      for (int64_t i = 0; i < fp8_bytes; ++i) ++h[(x[i] >> 3) & 15];
      for (int s = 0; s < 16; ++s) part[w][s] += h[s];
    }
  });
  for (int s = 0; s < 16; ++s) {
    hist[s] = 0;
    for (int w = 0; w < nt; ++w) hist[s] += part[w][s];
  }
  return MOE_OK;
} catch (const std::exception& ex) {
  set_error("moe_codec_histogram: %s", ex.what());
  return MOE_EINVAL;
}

extern "C" int64_t moe_codec_bound(int64_t record_bytes, int64_t fp8_bytes) {
  if (fp8_bytes <= 0 || fp8_bytes % kCodecBlock || record_bytes < fp8_bytes) return -1;
  const int64_t nblk = fp8_bytes / kCodecBlock;
  const int64_t b = nblk * kCodecMaxBlock + (record_bytes - fp8_bytes);
  return (b + 255) & ~int64_t{255};
}

extern "C" int64_t moe_codec_encode(const void* records, int64_t n_records, int64_t record_bytes,
                                    int64_t fp8_bytes, const uint8_t* code_lengths, void* dst,
                                    int64_t dst_capacity, int64_t* rec_offset,
                                    uint32_t* blk_offset, int32_t threads) try {
  if (!records || !code_lengths || !dst || !rec_offset || !blk_offset || n_records < 0 ||
      fp8_bytes <= 0 || fp8_bytes % kCodecBlock || record_bytes < fp8_bytes) {
    set_error("moe_codec_encode: bad arguments (fp8 bytes must be a positive multiple of %d)",
              kCodecBlock);
    return MOE_EINVAL;
  }
  CodeTable t;
  if (!make_codes(code_lengths, &t)) {
    set_error("moe_codec_encode: code lengths are not a prefix code of at most %d bits",
              kCodecMaxLen);
    return MOE_EINVAL;
  }
  const int64_t nblk = fp8_bytes / kCodecBlock;
  const int64_t tail = record_bytes - fp8_bytes;
  const int64_t bound = moe_codec_bound(record_bytes, fp8_bytes);
  // records are coded into per-record scratch in parallel, then packed in order
  const int nt = std::max(1, std::min<int>(threads, 64));
  std::vector<int64_t> size(n_records, 0);
  std::vector<std::vector<uint8_t>> scratch(nt, std::vector<uint8_t>(bound));
  uint8_t* out = static_cast<uint8_t*>(dst);
  int64_t cursor = 0;
  std::atomic<bool> failed{false};
  for (int64_t r0 = 0; r0 < n_records && !failed; r0 += nt) {
    const int64_t r1 = std::min<int64_t>(n_records, r0 + nt);
    run_threads(static_cast<int>(r1 - r0), [&](int k) {
      const int64_t r = r0 + k;
      uint8_t* buf = scratch[k].data();
      const uint8_t* x = static_cast<const uint8_t*>(records) + r * record_bytes;
      uint32_t* bo = blk_offset + r * (nblk + 1);
      int64_t o = 0;
      for (int64_t b = 0; b < nblk; ++b) {
        bo[b] = static_cast<uint32_t>(o);
        const int64_t n = encode_block(x + b * kCodecBlock, t, buf + o);
        if (n < 0) {
          failed = true;
          return;
        }
        o += n;
      }
      bo[nblk] = static_cast<uint32_t>(o);      // the raw tail
      memcpy(buf + o, x + fp8_bytes, tail);
      o += tail;
      size[r] = (o + 255) & ~int64_t{255};
    });
    if (failed) break;
    for (int64_t r = r0; r < r1; ++r) {
      if (cursor + size[r] > dst_capacity) {
        set_error("moe_codec_encode: destination of %lld bytes is too small",
                  (long long)dst_capacity);
        return MOE_EINVAL;
      }
      rec_offset[r] = cursor;
      memcpy(out + cursor, scratch[r - r0].data(), size[r]);
      cursor += size[r];
    }
  }
  if (failed) {
    set_error("moe_codec_encode: an exponent has no code (every length must be nonzero)");
    return MOE_EINVAL;
  }
  rec_offset[n_records] = cursor;
  return cursor;
} catch (const std::exception& ex) {
  set_error("moe_codec_encode: %s", ex.what());
  return MOE_EINVAL;
}

extern "C" int moe_codec_table(const uint8_t* code_lengths, uint16_t* lut) {
  MOE_REQUIRE(code_lengths && lut, "moe_codec_table: NULL pointer");
  CodeTable t;
  MOE_REQUIRE(make_codes(code_lengths, &t),
              "moe_codec_table: code lengths are not a prefix code of at most %d bits",
              kCodecMaxLen);
  // entry p: the two codes the stream bits p (least significant first) start
  // with: first symbol | second symbol << 4 | total length << 8
  uint8_t one[1 << kCodecMaxLen] = {0};        // code length << 4 | symbol
  for (int s = 0; s < 16; ++s) {
    const int l = t.len[s];
    if (!l) continue;
    for (int p = 0; p < (1 << kCodecMaxLen); ++p)
      if ((p & ((1 << l) - 1)) == t.rev[s]) one[p] = static_cast<uint8_t>((l << 4) | s);
  }
  for (int p = 0; p < kCodecLutSize; ++p) {
    const int e1 = one[p & ((1 << kCodecMaxLen) - 1)];
    const int l1 = e1 >> 4;
    const int e2 = one[(p >> l1) & ((1 << kCodecMaxLen) - 1)];
    lut[p] = static_cast<uint16_t>((e1 & 15) | ((e2 & 15) << 4) | ((l1 + (e2 >> 4)) << 8));
  }
  return MOE_OK;
}

extern "C" int moe_fetch_coded(const void* pool, const int64_t* rec_offset,
                               const uint32_t* blk_offset, int64_t record_bytes,
                               int64_t fp8_bytes, const uint16_t* lut,
                               const int32_t* fetch_expert, const int32_t* fetch_slot,
                               const int32_t* nmiss, int32_t max_jobs, void* cache,
                               int64_t slot_bytes, int32_t workgroups, void* stream) {
  MOE_REQUIRE(pool && rec_offset && blk_offset && lut && fetch_expert && fetch_slot && nmiss &&
                  cache, "moe_fetch_coded: NULL pointer");
  MOE_REQUIRE(fp8_bytes > 0 && fp8_bytes % kCodecBlock == 0 && record_bytes >= fp8_bytes &&
                  (record_bytes - fp8_bytes) % 16 == 0,
              "moe_fetch_coded: fp8 bytes must be a positive multiple of %d and the tail of 16",
              kCodecBlock);
  MOE_REQUIRE(slot_bytes >= record_bytes && slot_bytes % 16 == 0,
              "moe_fetch_coded: slots of at least one record, 16-byte multiples");
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(pool) % 256 == 0 &&
                  reinterpret_cast<uintptr_t>(cache) % 16 == 0,
              "moe_fetch_coded: pool 256-byte and cache 16-byte aligned");
  MOE_REQUIRE(max_jobs >= 1 && max_jobs <= 65535, "moe_fetch_coded: need 1 <= max_jobs <= 65535");
  MOE_REQUIRE(workgroups >= 1 && workgroups <= 65535,
              "moe_fetch_coded: need 1 <= workgroups <= 65535");
  hipLaunchKernelGGL(fetch_coded_kernel, dim3(workgroups), dim3(64 * kCodecWaves), 0,
                     as_stream(stream), static_cast<const uint8_t*>(pool), rec_offset, blk_offset,
                     static_cast<int32_t>(fp8_bytes / kCodecBlock), record_bytes - fp8_bytes, lut,
                     fetch_expert, fetch_slot, nmiss, max_jobs, static_cast<uint8_t*>(cache),
                     slot_bytes);
  return check_launch("moe_fetch_coded");
}

extern "C" int moe_route_fetch_coded(
    const void* x, const void* w, const float* bias, int32_t logit_dtype, int32_t hidden,
    int32_t n_experts, int32_t top_k, float* logits, int32_t* ids, float* weights,
    int32_t* slot_of, int32_t* slot_expert, int64_t* slot_stamp, int32_t cap, int64_t* step,
    int32_t* out_slot, int32_t* fetch_slot, int32_t* fetch_expert, int32_t* nmiss,
    int64_t* stats, const void* pool, const int64_t* rec_offset, const uint32_t* blk_offset,
    int64_t record_bytes, int64_t fp8_bytes, const uint16_t* lut, void* cache,
    int64_t slot_bytes, int32_t workgroups, void* stream) {
  MOE_REQUIRE(x && w && logits && ids && weights && slot_of && slot_expert && slot_stamp && step &&
                  out_slot && fetch_slot && fetch_expert && nmiss && pool && rec_offset &&
                  blk_offset && lut && cache,
              "moe_route_fetch_coded: NULL pointer");
  MOE_REQUIRE(logit_dtype == MOE_F32 || logit_dtype == MOE_BF16,
              "moe_route_fetch_coded: logit_dtype must be MOE_F32 or MOE_BF16");
  MOE_REQUIRE(hidden > 0 && hidden % 8 == 0, "moe_route_fetch_coded: hidden %% 8 != 0 (%d)",
              hidden);
  MOE_REQUIRE(top_k >= 1 && top_k <= kMaxTopK && top_k <= n_experts && n_experts <= 1024,
              "moe_route_fetch_coded: need 1 <= top_k <= min(32, n_experts), n_experts <= 1024");
  MOE_REQUIRE(cap >= 1 && cap <= 1024, "moe_route_fetch_coded: need 1 <= cap <= 1024");
  MOE_REQUIRE(top_k <= cap, "moe_route_fetch_coded: top_k (%d) exceeds the cache capacity (%d)",
              top_k, cap);
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0,
              "moe_route_fetch_coded: x and w must be 16-byte aligned");
  MOE_REQUIRE(fp8_bytes > 0 && fp8_bytes % kCodecBlock == 0 && record_bytes >= fp8_bytes &&
                  (record_bytes - fp8_bytes) % 16 == 0,
              "moe_route_fetch_coded: fp8 bytes must be a positive multiple of %d and the tail "
              "of 16", kCodecBlock);
  MOE_REQUIRE(slot_bytes >= record_bytes && slot_bytes % 16 == 0,
              "moe_route_fetch_coded: slots of at least one record, 16-byte multiples");
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(pool) % 256 == 0 &&
                  reinterpret_cast<uintptr_t>(cache) % 16 == 0,
              "moe_route_fetch_coded: pool 256-byte and cache 16-byte aligned");
  MOE_REQUIRE(workgroups >= 1 && workgroups <= 65535,
              "moe_route_fetch_coded: need 1 <= workgroups <= 65535");
  hipStream_t s = as_stream(stream);
  const int rc = launch_decode_logits(x, w, bias, hidden, n_experts,
                                      logit_dtype == MOE_BF16 ? 1 : 0, logits, step, s);
  if (rc) return rc;
  const auto* pl = static_cast<const uint8_t*>(pool);
  auto* ca = static_cast<uint8_t*>(cache);
  const int32_t nblk = static_cast<int32_t>(fp8_bytes / kCodecBlock);
  const int64_t tail = record_bytes - fp8_bytes;
#define MOE_RFC(PE, PC)                                                                         \
  hipLaunchKernelGGL((route_fetch_coded_kernel<PE, PC>), dim3(workgroups),                      \
                     dim3(64 * kCodecWaves), 0, s, logits, n_experts, top_k, ids, weights,      \
                     slot_of, slot_expert, slot_stamp, cap, step, out_slot, fetch_slot,         \
                     fetch_expert, nmiss, stats, pl, rec_offset, blk_offset, nblk, tail, lut,   \
                     ca, slot_bytes)
  if (n_experts <= 256) {
    if (cap <= 256) MOE_RFC(4, 4); else MOE_RFC(4, 16);
  } else {
    if (cap <= 256) MOE_RFC(16, 4); else MOE_RFC(16, 16);
  }
#undef MOE_RFC
  return check_launch("moe_route_fetch_coded(route+fetch)");
}
