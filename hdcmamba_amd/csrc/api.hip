// ABI version and status strings of libhdcmamba_hip.so.
#include <stdlib.h>

#include <atomic>

#include "hdcm_common.h"

thread_local HdcmTiming hdcm_timing_slot = {nullptr, nullptr, 0, 0};

extern "C" int hdcm_abi_version(void) { return HDCM_ABI_VERSION; }

// ------------------------------------------------------------------ launch options
namespace {

struct OptionInfo {
  const char* env;  // environment variable read when the library loads
  int dflt, lo, hi;
};
// index = hdcm_option value
constexpr OptionInfo kOptions[] = {
    {nullptr, 0, 0, 0},
    {"HDCM_SSM_SPIN_ROUNDS", 256, 0, 1 << 20},  // HDCM_OPT_SSM_SPIN_ROUNDS
    {"HDCM_SLOT_SEG_TILES", 0, 0, 1 << 20},     // HDCM_OPT_SLOT_SEG_TILES (0: automatic)
    {"HDCM_SKINNY_COLS8_MAX_N", 4096, 0, 1 << 30},  // HDCM_OPT_SKINNY_COLS8_MAX_N
    {"HDCM_SKINNY_FOLD_TAIL", 1, 0, 1},            // HDCM_OPT_SKINNY_FOLD_TAIL
    {"HDCM_STEP_SPIN_ROUNDS", 65536, 0, 1 << 24},  // HDCM_OPT_STEP_SPIN_ROUNDS
};
constexpr int kNumOptions = sizeof(kOptions) / sizeof(kOptions[0]);

std::atomic<int> g_options[kNumOptions];

int option_from_env(int k) {
  const OptionInfo& o = kOptions[k];
  const char* v = o.env ? getenv(o.env) : nullptr;
  if (!v || !*v) return o.dflt;
  char* end = nullptr;
  const long x = strtol(v, &end, 10);
  return (end && *end == '\0' && x >= o.lo && x <= o.hi) ? (int)x : o.dflt;
}

// runs when the library is loaded
struct OptionsAtLoad {
  OptionsAtLoad() {
    for (int k = 0; k < kNumOptions; ++k) g_options[k].store(option_from_env(k), std::memory_order_relaxed);
  }
} g_options_at_load;

}  // namespace

int hdcm_option_value(int option) {
  return (option > 0 && option < kNumOptions) ? g_options[option].load(std::memory_order_relaxed) : 0;
}

extern "C" int hdcm_set_option(int option, int value) {
  HDCM_CHECK_ARG(option > 0 && option < kNumOptions, HDCM_EINVAL);
  HDCM_CHECK_ARG(value >= kOptions[option].lo && value <= kOptions[option].hi, HDCM_EINVAL);
  g_options[option].store(value, std::memory_order_relaxed);
  return HDCM_OK;
}

extern "C" int hdcm_get_option(int option) { return hdcm_option_value(option); }

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
