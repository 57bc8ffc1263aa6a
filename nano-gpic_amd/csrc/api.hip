// Library identification and status messages of libgpic_fp8.so.
#include "gpic_launch.h"

extern "C" {

const char *gpic_fp8_version(void) { return "gpic_fp8 0.1 gfx950"; }

const char *gpic_fp8_status_string(int status) {
  switch (status) {
    case GPIC_OK: return "ok";
    case GPIC_EINVAL: return "invalid argument (null pointer or negative size)";
    case GPIC_EDTYPE: return "unsupported dtype";
    case GPIC_ESHAPE: return "unsupported shape or leading dimension (alignment rules: multiples of 16 / 8)";
    case GPIC_EALIGN: return "pointer not 16-byte aligned";
    case GPIC_EWORKSPACE: return "workspace too small";
    default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown status";
  }
}

}  // extern "C"
