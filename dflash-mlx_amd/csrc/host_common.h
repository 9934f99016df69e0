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

}  // namespace dflash
