// Error reporting, version and host-pool entry points of the C ABI.
#include "common.hpp"

#include <dlfcn.h>
#include <string.h>

namespace moe {

static thread_local char g_err[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return MOE_OK;
}

// For each bit pattern u of [first, first + count): the conversion unit's
// packed e4m3x4 of (u, u with the sign flipped, u ^ 0x00400001, ~u) against
// four f32_to_e4m3 calls; every mismatching pattern adds one to *mismatches.
__global__ __launch_bounds__(256) void e4m3_check_kernel(uint32_t first, uint32_t count,
                                                         unsigned long long* mismatches) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  const uint32_t u = first + i;
  const uint32_t us[4] = {u, u ^ 0x80000000u, u ^ 0x00400001u, ~u};
  float v[4];
  uint32_t want = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[k] = __builtin_bit_cast(float, us[k]);
    want |= f32_to_e4m3(v[k]) << (8 * k);
  }
  if (e4m3x4(v[0], v[1], v[2], v[3]) != want) atomicAdd(mismatches, 1ull);
}

// out[i] = silu_mul(g[i], u[i]), the expert kernels' SiLU(gate) * up.
__global__ __launch_bounds__(256) void silu_check_kernel(const float* __restrict__ g,
                                                         const float* __restrict__ u,
                                                         float* __restrict__ out, uint32_t n) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = silu_mul(g[i], u[i]);
}

// Read n16 16-byte words of src once each (grid-stride, U nontemporal loads
// in flight per lane) and fold them into one XOR per lane; a lane writes only
// if its XOR equals `never`, so the loads cannot be dropped and almost
// nothing is written.
template <int U>
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ src,
                                                          int64_t n16, uint32_t never,
                                                          uint32_t* __restrict__ sink) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (U - 1) * stride < n16; i += U * stride) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == never) sink[0] = acc;
}

}  // namespace moe

extern "C" {

int moe_stream_read(const void* src, int64_t bytes, int32_t workgroups, uint32_t* sink,
                    void* stream) {
  MOE_REQUIRE(src && sink, "moe_stream_read: NULL pointer");
  MOE_REQUIRE(bytes > 0 && bytes % 16 == 0, "moe_stream_read: bytes must be a positive multiple "
              "of 16");
  MOE_REQUIRE(reinterpret_cast<uintptr_t>(src) % 16 == 0, "moe_stream_read: src must be 16-byte "
              "aligned");
  MOE_REQUIRE(workgroups >= 1 && workgroups <= 65535, "moe_stream_read: need 1 <= workgroups "
              "<= 65535");
  hipLaunchKernelGGL(moe::stream_read_kernel<4>, dim3(workgroups), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const moe::u32x4*>(src),
                     bytes / 16, 0x9e3779b9u, sink);
  return moe::check_launch("moe_stream_read");
}

int moe_e4m3_check(uint32_t first, uint32_t count, uint64_t* mismatches, void* stream) {
  MOE_REQUIRE(mismatches != nullptr, "moe_e4m3_check: mismatches is NULL");
  MOE_REQUIRE(count >= 1 && count <= (1u << 30), "moe_e4m3_check: need 1 <= count <= 2^30");
  MOE_REQUIRE(static_cast<uint64_t>(first) + count <= (1ull << 32),
              "moe_e4m3_check: range past 2^32");
  hipLaunchKernelGGL(moe::e4m3_check_kernel, dim3((count + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), first, count,
                     reinterpret_cast<unsigned long long*>(mismatches));
  return moe::check_launch("moe_e4m3_check");
}

int moe_silu_check(const float* g, const float* u, float* out, uint32_t n, void* stream) {
  if (n == 0) return MOE_OK;
  MOE_REQUIRE(g && u && out, "moe_silu_check: NULL pointer");
  MOE_REQUIRE(n <= (1u << 30), "moe_silu_check: need n <= 2^30");
  hipLaunchKernelGGL(moe::silu_check_kernel, dim3((n + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), g, u, out, n);
  return moe::check_launch("moe_silu_check");
}

const char* moe_last_error(void) { return moe::g_err; }

const char* moe_version(void) { return "moeoffload 0.1 gfx950"; }

const char* moe_hip_runtime_path(void) {
  static char path[1024] = "";
  Dl_info info;
  void* sym = reinterpret_cast<void*>(&hipGetLastError);
  if (dladdr(sym, &info) && info.dli_fname) {
    strncpy(path, info.dli_fname, sizeof(path) - 1);
  }
  return path;
}

int moe_host_alloc(void** host_ptr, size_t bytes, int flags) {
  MOE_REQUIRE(host_ptr != nullptr, "moe_host_alloc: host_ptr is NULL");
  MOE_REQUIRE(bytes > 0, "moe_host_alloc: zero bytes");
  MOE_REQUIRE(flags == 0 || flags == 1, "moe_host_alloc: flags must be 0 or 1");
  unsigned f = hipHostMallocMapped | (flags ? hipHostMallocNonCoherent : hipHostMallocCoherent);
  hipError_t e = hipHostMalloc(host_ptr, bytes, f);
  if (e != hipSuccess) {
    moe::set_error("moe_host_alloc(%zu B): %s", bytes, hipGetErrorString(e));
    *host_ptr = nullptr;
    return static_cast<int>(e);
  }
  return MOE_OK;
}

int moe_host_free(void* host_ptr) {
  if (host_ptr == nullptr) return MOE_OK;
  hipError_t e = hipHostFree(host_ptr);
  if (e != hipSuccess) {
    moe::set_error("moe_host_free: %s", hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return MOE_OK;
}

int moe_device_ptr_of(const void* host_ptr, void** dev_ptr) {
  MOE_REQUIRE(host_ptr != nullptr && dev_ptr != nullptr, "moe_device_ptr_of: NULL argument");
  hipPointerAttribute_t attr;
  hipError_t e = hipPointerGetAttributes(&attr, host_ptr);
  if (e != hipSuccess || attr.type != hipMemoryTypeHost) {
    (void)hipGetLastError();  // clear the sticky error of a failed query
    moe::set_error("moe_device_ptr_of: %p is not page-locked host memory "
                   "(expected a contiguous page-locked CPU buffer)", host_ptr);
    return MOE_EINVAL;
  }
  void* d = nullptr;
  e = hipHostGetDevicePointer(&d, const_cast<void*>(host_ptr), 0);
  if (e != hipSuccess) {
    moe::set_error("moe_device_ptr_of: hipHostGetDevicePointer: %s", hipGetErrorString(e));
    return static_cast<int>(e);
  }
  *dev_ptr = d;
  return MOE_OK;
}

}  // extern "C"
