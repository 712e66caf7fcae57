// Library-wide C-ABI entry points (no device code).
#include "../../include/mskv.h"

extern "C" int mskv_version(void) { return 100; }  // 0.1.0

extern "C" const char* mskv_status_string(int status) {
  switch (status) {
    case MSKV_OK: return "ok";
    case MSKV_EINVAL: return "invalid argument (null pointer, bad size or inconsistent shape)";
    case MSKV_EUNSUPPORTED: return "shape not supported by the gfx950 kernels";
    case MSKV_EWORKSPACE: return "workspace missing or too small";
    default: return status > 0 ? "HIP launch error" : "unknown status";
  }
}
