// Library-level C ABI entry points: error text and version.
#include <hip/hip_runtime.h>

#include "respect_amd.h"

extern "C" const char* rspx_strerror(int code) {
  switch (code) {
    case RSPX_OK: return "ok";
    case RSPX_EINVAL: return "invalid size, stride or null pointer";
    case RSPX_EUNSUPPORTED: return "unsupported head_dim, GQA ratio or dtype";
    case RSPX_EWORKSPACE: return "workspace missing or too small";
    case RSPX_EALIGN: return "pointer or stride not 16-byte aligned";
    case RSPX_ELAUNCH: return "HIP kernel launch failed";
    default: return "unknown error";
  }
}

extern "C" const char* rspx_version(void) { return "respect_amd 0.1.0 gfx950"; }
