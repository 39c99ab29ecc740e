// The selective scan of ssm.hip without a caller workspace, for callers that cannot allocate
// device memory (code under HIP graph capture, serving loops, harnesses that forbid it).
//
// hdcm_ssm_fwd_noalloc runs the kernels of hdcm_ssm_fwd on `scratch`, a file-scope device
// array of HDCM_SSM_NOALLOC_SCRATCH_BYTES, instead of a caller workspace.  Each GPU the
// library runs on holds its own copy of the array (until the process ends) at its own
// address.  That address is looked up once per device, on the first call that runs on the
// device, with the device current (hipGetSymbolAddress), and host code passes only it to the
// kernels: the array's name is a host-side stand-in, not a device address.  The array starts
// at zero when the library is loaded, which is the state the scan's workspace needs before
// its first call; after that the kernel keeps it consistent itself (its call counter, and
// tile totals tagged with it), so nothing is cleared between calls.  Calls that overlap on
// one GPU share its array and race.
#include <mutex>

#include "hdcm_common.h"

static __device__ __align__(256) unsigned char scratch[HDCM_SSM_NOALLOC_SCRATCH_BYTES];

// ssm.hip
int hdcm_ssm_check_fwd(const void* projs, int64_t proj_row_stride, const void* A_log, const void* y,
                       int64_t y_row_stride, const float* row_stats, int64_t stats_part_stride, int64_t B,
                       int64_t L, int64_t ds, int dtype);
int hdcm_ssm_launch_fwd(const void* projs, int64_t proj_row_stride, const void* A_log, const float* h0, void* y,
                        int64_t y_row_stride, float* h_final, float* row_stats, int64_t stats_part_stride, void* ws,
                        int64_t B, int64_t L, int64_t ds, int dtype, hipStream_t s);

namespace {

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_addr[kMaxDevices];  // per device; null until looked up

// The device `s` runs on, and that device's address of `scratch`.
int scratch_for_stream(hipStream_t s, void** out) {
  int dev = 0;
  const hipError_t ge = s == nullptr ? hipGetDevice(&dev) : hipStreamGetDevice(s, &dev);
  if (ge != hipSuccess) return HDCM_ELAUNCH;
  if (dev < 0 || dev >= kMaxDevices) return HDCM_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_addr[dev] == nullptr) {
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return HDCM_ELAUNCH;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return HDCM_ELAUNCH;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || p == nullptr) return HDCM_ELAUNCH;
    scratch_addr[dev] = p;
  }
  *out = scratch_addr[dev];
  return HDCM_OK;
}

}  // namespace

extern "C" int hdcm_ssm_fwd_noalloc(const void* projs, int64_t proj_row_stride, const void* A_log,
                                    const float* h0, void* y, int64_t y_row_stride, float* h_final,
                                    float* row_stats, int64_t stats_part_stride, int64_t B, int64_t L, int64_t ds,
                                    int dtype, void* stream) {
  int st = hdcm_ssm_check_fwd(projs, proj_row_stride, A_log, y, y_row_stride, row_stats, stats_part_stride, B, L, ds,
                              dtype);
  if (st) return st;
  if (B == 0 || L == 0) return HDCM_OK;
  HDCM_CHECK_ARG(hdcm_ssm_workspace_bytes(B, L, ds) <= HDCM_SSM_NOALLOC_SCRATCH_BYTES, HDCM_ETOOBIG);
  hipStream_t s = (hipStream_t)stream;
  void* ws = nullptr;
  st = scratch_for_stream(s, &ws);
  if (st) return st;
  return hdcm_ssm_launch_fwd(projs, proj_row_stride, A_log, h0, y, y_row_stride, h_final, row_stats,
                             stats_part_stride, ws, B, L, ds, dtype, s);
}
