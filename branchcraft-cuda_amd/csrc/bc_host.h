// Host-side helpers shared by the launch code of the kernel files.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>

namespace bch {

// Compute units of the current device, cached per device (an immutable
// attribute, so the cache is safe to share between threads).  256 when the
// query fails.
inline int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64) {
    const int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n < 1)
    n = 256;
  if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace bch
