// Library-level entry points of the C-ABI (version and status strings).
#include "xk_common.h"

extern "C" const char* xk_version(void) { return "xk 0.1.0 gfx950"; }

extern "C" const char* xk_status_string(int status) {
  switch (status) {
    case XK_OK:
      return "ok";
    case XK_ERR_INVALID:
      return "invalid argument";
    case XK_ERR_UNSUPPORTED:
      return "unsupported dtype or configuration";
    case XK_ERR_WORKSPACE:
      return "workspace missing or too small";
    case XK_ERR_SCRATCH:
      return "problem needs more memory than the static scratch buffer holds";
    default:
      return status > 0 ? hipGetErrorString(static_cast<hipError_t>(status))
                        : "unknown error";
  }
}
