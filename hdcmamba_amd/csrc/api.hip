// ABI version and status strings of libhdcmamba_hip.so.
#include "hdcm_common.h"

thread_local HdcmTiming hdcm_timing_slot = {nullptr, nullptr, 0, 0};

extern "C" int hdcm_abi_version(void) { return HDCM_ABI_VERSION; }

extern "C" int hdcm_time_launches(void* const* start_events, void* const* stop_events, int n) {
  HDCM_CHECK_ARG(n >= 0 && (n == 0 || (start_events && stop_events)), HDCM_EINVAL);
  for (int k = 0; k < n; ++k) HDCM_CHECK_ARG(start_events[k] && stop_events[k], HDCM_EINVAL);
  hdcm_timing_slot = {n ? start_events : nullptr, n ? stop_events : nullptr, n, 0};
  return HDCM_OK;
}

extern "C" int hdcm_timed_launch_count(void) { return hdcm_timing_slot.used; }

extern "C" const char* hdcm_strerror(int status) {
  switch (status) {
    case HDCM_OK: return "ok";
    case HDCM_EINVAL: return "invalid argument (null pointer, shape or stride)";
    case HDCM_EALIGN: return "pointer or row stride is not 16-byte aligned";
    case HDCM_EUNSUPPORTED: return "unsupported dtype/shape combination";
    case HDCM_ELAUNCH: return "HIP kernel launch failed";
    case HDCM_EWORKSPACE: return "workspace missing or too small";
    case HDCM_ETOOBIG: return "input exceeds the fixed scratch of the no-allocation entry point";
    default: return "unknown hdcm status";
  }
}
