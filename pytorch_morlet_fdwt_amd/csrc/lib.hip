// Library-level C ABI helpers: error strings and the build tag.
#include "common.h"

extern "C" const char* fdwt_error_string(int code) {
  switch (code) {
    case 0: return "success";
    case FDWT_ERR_ARG: return "fdwt: invalid argument (size, mode, dtype, filter length or pointer)";
    case FDWT_ERR_TOO_LONG: return "fdwt: row too long for the kernel's on-chip buffers";
    case FDWT_ERR_SCRATCH: return "fdwt: call too large for the no-allocation entry's fixed scratch";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "fdwt: unknown error";
}

extern "C" const char* fdwt_version(void) { return "fdwt-hip 0.1 gfx950"; }
