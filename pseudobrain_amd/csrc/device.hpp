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

// Whether a decode call's state (at `state`, `moved` bytes read and written)
// is likely still in the last-level cache: the previous decode call on this
// device stepped the same pool and the call moves at most cache_bytes. A
// model's layers each keep their own pool, so their consecutive calls alternate
// pools and stream; a loop stepping one pool keeps it cached. Records `state`
// for the next call.
bool state_likely_cached(const void *state, long moved, long cache_bytes);

// Raises `kernel`'s dynamic LDS limit to `bytes` on the current device, once
// per device (`flags`: MAX_DEVICES entries kept by the caller); false when the
// runtime refuses.
bool smem_configured(const void *kernel, size_t bytes, std::atomic<bool> *flags);

}  // namespace pbgdn
