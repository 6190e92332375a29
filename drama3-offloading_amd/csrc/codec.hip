// Entropy-coded expert records: fewer bytes over the host link, decoded on
// the GPU into byte-exact cache slots.
//
// The fp8 (e4m3) weights of a record are 1 sign, 4 exponent and 3 mantissa
// bits.  Block-scaled weights use few exponents (the 128x128 block maximum
// maps to 448), so the exponent nibble carries about 2.6 bits; sign and
// mantissa are close to uniform.  A record's fp8 bytes are cut into blocks
// of 8192 and each block is stored as
//
//   [0, 4096)        nibble plane: byte j = nib(x[2j]) | nib(x[2j+1]) << 4,
//                    nib(x) = (sign << 3) | mantissa
//   [4096, 4160)     lane header: byte l = length in bytes of stream l
//   [4160, ...)      64 streams, stream l the exponents of x[128l, 128l+128)
//                    as canonical Huffman codes (at most 8 bits), written
//                    least significant bit first, each stream byte-padded
//   padded to 16 bytes.
//
// The bytes after the fp8 part (the block scales) follow raw.  Records are
// 256-byte aligned in the coded pool; where each record and each of its
// blocks starts is a device-resident index, so the fetch kernel needs no
// host read to find them.
//
// Decoding: one wave per block.  The header and streams go to LDS, the
// nibble plane straight to registers (lane l takes bytes 64l..64l+63); each
// lane finds its stream's start with a wave prefix sum of the header, then
// decodes its 128 exponents with a 256-entry table (8 peeked bits -> symbol
// and code length) in LDS and writes its 128 bytes to the cache slot.
#include <string.h>

#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

#include "common.hpp"

namespace moe {

constexpr int kCodecBlock = 8192;                 // fp8 bytes per block
constexpr int kCodecLanes = 64;
constexpr int kCodecPerLane = kCodecBlock / kCodecLanes;   // 128 symbols
constexpr int kCodecPlane = kCodecBlock / 2;      // nibble plane bytes
constexpr int kCodecHeader = kCodecLanes;         // one length byte per lane
constexpr int kCodecMaxLen = 8;                   // longest code, bits
constexpr int kCodecMaxBlock = kCodecPlane + kCodecHeader + kCodecBlock + 16;

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

// Fetch of coded records: job j copies coded record fetch_expert[j] of the
// pool into cache slot fetch_slot[j], decoded; j < *nmiss (read on the
// device).  Units are (job, block) pairs plus one per job for the raw tail,
// dealt to the waves of the grid round-robin.
__global__ __launch_bounds__(64 * kCodecWaves) void fetch_coded_kernel(
    const uint8_t* __restrict__ pool, const int64_t* __restrict__ rec_off,
    const uint32_t* __restrict__ blk_off, int32_t nblk, int64_t tail,
    const uint8_t* __restrict__ lut_g, const int32_t* __restrict__ fexp,
    const int32_t* __restrict__ fslot, const int32_t* __restrict__ nmiss, int32_t max_jobs,
    uint8_t* __restrict__ cache, int64_t slot_bytes) {
  __shared__ __align__(16) uint8_t lds[kCodecWaves][kCodecLds];
  __shared__ uint8_t lut[256];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  lut[threadIdx.x] = lut_g[threadIdx.x];          // 256 threads
  __syncthreads();
  const int32_t nm = min(*nmiss, max_jobs);
  const int64_t per_job = static_cast<int64_t>(nblk) + 1;
  const int64_t units = static_cast<int64_t>(nm) * per_job;
  const uint32_t* w32 = reinterpret_cast<const uint32_t*>(lds[wave]);
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * kCodecWaves + wave; u < units;
       u += static_cast<int64_t>(gridDim.x) * kCodecWaves) {
    const int64_t j = u / per_job;
    const int b = static_cast<int>(u - j * per_job);
    const int64_t e = fexp[j];
    const int64_t sl = fslot[j];
    const uint32_t* bo = blk_off + e * per_job;
    const uint8_t* src = pool + rec_off[e] + bo[b];
    uint8_t* dst = cache + sl * slot_bytes + static_cast<int64_t>(b) * kCodecBlock;
    if (b == nblk) {                              // the raw tail (block scales)
      for (int64_t i = lane * 16; i < tail; i += 64 * 16)
        *reinterpret_cast<u32x4*>(dst + i) = *reinterpret_cast<const u32x4*>(src + i);
      continue;
    }
    // nibble plane: this lane's 64 bytes (its 128 symbols) straight to registers
    u32x4 nv[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      nv[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + 64 * lane) + k);
    // header and streams to this wave's LDS
    const int rest = static_cast<int>(bo[b + 1] - bo[b]) - kCodecPlane;   // multiple of 16
    for (int i = lane * 16; i < rest; i += 64 * 16)
      *reinterpret_cast<u32x4*>(&lds[wave][i]) =
          __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + kCodecPlane + i));
    const int start = kCodecHeader + wave_exclusive_sum(lds[wave][lane]);
    // LSB-first bit reader over this lane's stream
    int wi = start >> 2;
    uint64_t buf = static_cast<uint64_t>(w32[wi++]) >> ((start & 3) * 8);
    int nbits = 32 - (start & 3) * 8;
    const uint32_t nw[16] = {nv[0].x, nv[0].y, nv[0].z, nv[0].w, nv[1].x, nv[1].y, nv[1].z, nv[1].w,
                             nv[2].x, nv[2].y, nv[2].z, nv[2].w, nv[3].x, nv[3].y, nv[3].z, nv[3].w};
    uint32_t ow[32];
#pragma unroll
    for (int i = 0; i < kCodecPerLane; ++i) {
      if (nbits < kCodecMaxLen) {
        buf |= static_cast<uint64_t>(w32[wi++]) << nbits;
        nbits += 32;
      }
      const uint32_t ent = lut[buf & 255];
      const uint32_t len = ent >> 4;
      buf >>= len;
      nbits -= static_cast<int>(len);
      const uint32_t nib = (nw[i >> 3] >> ((i & 7) * 4)) & 15;
      const uint32_t byte = ((nib & 8) << 4) | ((ent & 15) << 3) | (nib & 7);
      if ((i & 3) == 0)
        ow[i >> 2] = byte;
      else
        ow[i >> 2] |= byte << ((i & 3) * 8);
    }
    u32x4* d = reinterpret_cast<u32x4*>(dst + kCodecPerLane * lane);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      d[k] = u32x4{ow[4 * k], ow[4 * k + 1], ow[4 * k + 2], ow[4 * k + 3]};
  }
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
  for (int j = 0; j < kCodecPlane; ++j)
    out[j] = static_cast<uint8_t>(nib_of(x[2 * j]) | (nib_of(x[2 * j + 1]) << 4));
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
  while (n & 15) out[n++] = 0;
  return n;
}

}  // namespace moe

using namespace moe;

extern "C" int moe_codec_histogram(const void* records, int64_t n_records, int64_t record_bytes,
                                   int64_t fp8_bytes, uint64_t* hist, int32_t threads) {
  MOE_REQUIRE(records && hist, "moe_codec_histogram: NULL pointer");
  MOE_REQUIRE(n_records >= 0 && fp8_bytes >= 0 && fp8_bytes <= record_bytes,
              "moe_codec_histogram: bad sizes");
  const int nt = std::max(1, std::min<int>(threads, 64));
  std::vector<std::vector<uint64_t>> part(nt, std::vector<uint64_t>(16, 0));
  std::vector<std::thread> pool;
  for (int w = 0; w < nt; ++w) {
    pool.emplace_back([&, w] {
      for (int64_t r = w; r < n_records; r += nt) {
        const uint8_t* x = static_cast<const uint8_t*>(records) + r * record_bytes;
        uint64_t h[16] = {0};
        for (int64_t i = 0; i < fp8_bytes; ++i) ++h[(x[i] >> 3) & 15];
        for (int s = 0; s < 16; ++s) part[w][s] += h[s];
      }
    });
  }
  for (auto& th : pool) th.join();
  for (int s = 0; s < 16; ++s) {
    hist[s] = 0;
    for (int w = 0; w < nt; ++w) hist[s] += part[w][s];
  }
  return MOE_OK;
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
                                    uint32_t* blk_offset, int32_t threads) {
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
    std::vector<std::thread> pool;
    for (int64_t r = r0; r < r1; ++r) {
      pool.emplace_back([&, r] {
        uint8_t* buf = scratch[r - r0].data();
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
    }
    for (auto& th : pool) th.join();
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
}

extern "C" int moe_codec_table(const uint8_t* code_lengths, uint8_t* lut) {
  MOE_REQUIRE(code_lengths && lut, "moe_codec_table: NULL pointer");
  CodeTable t;
  MOE_REQUIRE(make_codes(code_lengths, &t),
              "moe_codec_table: code lengths are not a prefix code of at most %d bits",
              kCodecMaxLen);
  for (int p = 0; p < 256; ++p) lut[p] = 0;
  for (int s = 0; s < 16; ++s) {
    const int l = t.len[s];
    if (!l) continue;
    for (int p = 0; p < 256; ++p)
      if ((p & ((1 << l) - 1)) == t.rev[s]) lut[p] = static_cast<uint8_t>((l << 4) | s);
  }
  return MOE_OK;
}

extern "C" int moe_fetch_coded(const void* pool, const int64_t* rec_offset,
                               const uint32_t* blk_offset, int64_t record_bytes,
                               int64_t fp8_bytes, const uint8_t* lut,
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
