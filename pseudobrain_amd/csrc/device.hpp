// The shape of the GPU a call runs on, queried from the runtime (not assumed):
// compute units, and XCDs (accelerator complex dies, each with its own L2;
// workgroups are dispatched round-robin over them).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>

namespace pbgdn {

struct DeviceShape {
  int cus;   // compute units available to this process (a partitioned GPU shows its share)
  int xcds;  // XCDs those compute units are spread over
};

constexpr int MAX_DEVICES = 64;

// The current device's ordinal, or -1 when it cannot be read (or is beyond
// MAX_DEVICES).
int current_device();

// The current device's shape, queried once per device; false when the runtime
// cannot report it.
bool device_shape(DeviceShape &out);

// Raises `kernel`'s dynamic LDS limit to `bytes` on the current device, once
// per device (`flags`: MAX_DEVICES entries kept by the caller); false when the
// runtime refuses.
bool smem_configured(const void *kernel, size_t bytes, std::atomic<bool> *flags);

// Debug build (PBGDN_DEBUG, libpbgdn_debug.so): the entry points fill their
// pure outputs and workspaces with 0xff bytes (a NaN in float32, bfloat16 and
// float16) on the stream before launching, so that an element no kernel
// writes stays NaN; in-place buffers (state pools, carried tails) are left
// alone. Nothing in a normal build.
#ifdef PBGDN_DEBUG
inline void debug_poison(void *p, size_t bytes, hipStream_t st) {
  if (p && bytes) (void)hipMemsetAsync(p, 0xff, bytes, st);
}
#else
inline void debug_poison(void *, size_t, hipStream_t) {}
#endif

}  // namespace pbgdn
