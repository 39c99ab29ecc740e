// fp32 instantiations of the slot memory's plain attention pass (hdcm_slot_attend_fwd is in
// slot_attend.hip).
#include "slot_kernels.h"

int hdcm_slot::attend_launch_f32(const void* base, int64_t row_stride, int64_t q_col, int64_t k_col,
                                 int64_t v_col, const void* gamma, int phi, void* ws, void* out,
                                 int64_t out_row_stride, int64_t out_col, const void* chain,
                                 int64_t chain_row_stride, int64_t B, int64_t L, int64_t H, int64_t C,
                                 const SlotPlan& pl, hipStream_t s) {
  int st;
#define HDCM_ATTEND_CASE(TT, HDV, PH)                                                                          \
  if (pl.HD == HDV && (phi != 0) == PH) {                                                                    \
    st = launch_state<TT, HDV, PH>(base, row_stride, k_col, v_col - k_col, gamma, nullptr, ws, B, L, H, pl, s); \
    if (st) return st;                                                                                       \
    if (chain)                                                                                               \
      return launch_gate<TT, HDV, PH, false, true>(base, row_stride, q_col, k_col - q_col, v_col - q_col, 0,  \
                                                   gamma, nullptr, nullptr, 0.f, ws, out, out_row_stride,    \
                                                   out_col, nullptr, nullptr, 0, B, L, H, C, pl, s, chain,   \
                                                   chain_row_stride);                                        \
    return launch_gate<TT, HDV, PH, false>(base, row_stride, q_col, k_col - q_col, v_col - q_col, 0, gamma,   \
                                           nullptr, nullptr, 0.f, ws, out, out_row_stride, out_col, nullptr, \
                                           nullptr, 0, B, L, H, C, pl, s);                                  \
  }
  HDCM_ATTEND_CASE(float, 16, true)
  HDCM_ATTEND_CASE(float, 32, true)
  HDCM_ATTEND_CASE(float, 48, true)
  HDCM_ATTEND_CASE(float, 64, true)
  HDCM_ATTEND_CASE(float, 80, true)
  HDCM_ATTEND_CASE(float, 96, true)
  HDCM_ATTEND_CASE(float, 112, true)
  HDCM_ATTEND_CASE(float, 128, true)
  HDCM_ATTEND_CASE(float, 16, false)
  HDCM_ATTEND_CASE(float, 32, false)
  HDCM_ATTEND_CASE(float, 48, false)
  HDCM_ATTEND_CASE(float, 64, false)
  HDCM_ATTEND_CASE(float, 80, false)
  HDCM_ATTEND_CASE(float, 96, false)
  HDCM_ATTEND_CASE(float, 112, false)
  HDCM_ATTEND_CASE(float, 128, false)
#undef HDCM_ATTEND_CASE
  return HDCM_EUNSUPPORTED;
}
