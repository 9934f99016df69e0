// ABI handshake and error text of libdflash_gfx950.so.
#include "dflash_gdn.h"

#include <hip/hip_runtime.h>

extern "C" int dflash_abi_version(void) { return DFLASH_ABI_VERSION; }

extern "C" const char* dflash_strerror(int code) {
  switch (code) {
    case DFLASH_OK: return "ok";
    case DFLASH_ERR_NULL: return "a required pointer is NULL";
    case DFLASH_ERR_SHAPE: return "a size is out of range or inconsistent";
    case DFLASH_ERR_UNSUPPORTED: return "head dimension or dtype not supported by this build";
    case DFLASH_ERR_ALIGN: return "pointer or stride misaligned for vector access";
    case DFLASH_ERR_WORKSPACE: return "workspace smaller than required";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "unknown dflash error";
}
