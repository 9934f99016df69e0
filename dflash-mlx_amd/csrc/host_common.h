// Host-side helpers shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dflash_gdn.h"

namespace dflash {

// Layers whose pointers travel in one launch's kernel arguments.  Longer
// lists are split into several launches.
constexpr int kMaxLayersPerLaunch = 32;

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline int to_status(hipError_t e) { return e == hipSuccess ? DFLASH_OK : (int)e; }

// Compute units of the current device (cached per device; 0 if unknown).
inline int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

}  // namespace dflash
