// Per-device queries of the GPU's shape (device.hpp) and the streaming
// bandwidth probe (pbgdn_stream_probe).
#include "device.hpp"

#include <atomic>

#include "common.hpp"
#include "pbgdn.h"

namespace pbgdn {

int current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return -1;
  return dev;
}

bool device_shape(DeviceShape &out) {
  // Packed (cus << 16 | xcds) per device; 0 until queried. Racing first calls
  // query the same values, so either store is right.
  static std::atomic<int> cache[MAX_DEVICES];
  const int dev = current_device();
  if (dev < 0) return false;
  int packed = cache[dev].load(std::memory_order_relaxed);
  if (packed == 0) {
    int cus = 0, xcds = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return false;
    if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || xcds <= 0) xcds = 1;
    if (cus >= (1 << 15) || xcds >= (1 << 15)) return false;
    packed = (cus << 16) | xcds;
    cache[dev].store(packed, std::memory_order_relaxed);
  }
  out.cus = packed >> 16;
  out.xcds = packed & 0xffff;
  return true;
}

bool smem_configured(const void *kernel, size_t bytes, std::atomic<bool> *flags) {
  const int dev = current_device();
  if (dev < 0) return false;
  if (flags[dev].load(std::memory_order_acquire)) return true;
  // racing first calls set the same attribute: idempotent
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)) != hipSuccess) {
    return false;
  }
  flags[dev].store(true, std::memory_order_release);
  return true;
}

namespace {

// Streaming copy: 16-byte buffer loads then stores, UNITS pieces of 16 bytes
// per thread in flight, grid-stride, non-temporal (nt) on both sides.
constexpr int PROBE_UNITS = 4;
constexpr int PROBE_NT = 256;

__global__ __launch_bounds__(PROBE_NT) void stream_probe_kernel(const unsigned char *src, unsigned char *dst,
                                                                uint32_t bytes) {
  const __amdgpu_buffer_rsrc_t rs = rsrc(src, bytes), rd = rsrc(dst, bytes);
  constexpr uint32_t BLOCK = PROBE_NT * 16u * PROBE_UNITS;
  const uint32_t stride = gridDim.x * BLOCK;
  for (uint32_t base = blockIdx.x * BLOCK; base < bytes; base += stride) {
    v4u32_t x[PROBE_UNITS];
#pragma unroll
    for (int u = 0; u < PROBE_UNITS; ++u)
      x[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, base + (u * PROBE_NT + threadIdx.x) * 16u, 0, 2);
#pragma unroll
    for (int u = 0; u < PROBE_UNITS; ++u)
      __builtin_amdgcn_raw_buffer_store_b128(x[u], rd, base + (u * PROBE_NT + threadIdx.x) * 16u, 0, 2);
  }
}

}  // namespace
}  // namespace pbgdn

extern "C" int pbgdn_stream_probe(const void *src, void *dst, int64_t bytes, void *stream) {
  if (bytes < 0 || bytes % 16 != 0 || bytes > (int64_t{1} << 31) - 16) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  if (bytes == 0) return PBGDN_OK;
  if (!src || !dst || (reinterpret_cast<uintptr_t>(src) & 15u) || (reinterpret_cast<uintptr_t>(dst) & 15u)) {
    return PBGDN_ERR_INVALID_ARGUMENT;
  }
  pbgdn::DeviceShape shape;
  if (!pbgdn::device_shape(shape)) return PBGDN_ERR_LAUNCH;
  hipLaunchKernelGGL(pbgdn::stream_probe_kernel, dim3(static_cast<unsigned>(shape.cus) * 16u),
                     dim3(pbgdn::PROBE_NT), 0, static_cast<hipStream_t>(stream),
                     static_cast<const unsigned char *>(src), static_cast<unsigned char *>(dst),
                     static_cast<uint32_t>(bytes));
  return hipGetLastError() == hipSuccess ? PBGDN_OK : PBGDN_ERR_LAUNCH;
}
