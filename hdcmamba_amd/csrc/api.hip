// ABI version and status strings of libhdcmamba_hip.so.
#include "hdcm_common.h"

extern "C" int hdcm_abi_version(void) { return HDCM_ABI_VERSION; }

extern "C" const char* hdcm_strerror(int status) {
  switch (status) {
    case HDCM_OK: return "ok";
    case HDCM_EINVAL: return "invalid argument (null pointer, shape or stride)";
    case HDCM_EALIGN: return "pointer or row stride is not 16-byte aligned";
    case HDCM_EUNSUPPORTED: return "unsupported dtype/shape combination";
    case HDCM_ELAUNCH: return "HIP kernel launch failed";
    case HDCM_EWORKSPACE: return "workspace missing or too small";
    default: return "unknown hdcm status";
  }
}
