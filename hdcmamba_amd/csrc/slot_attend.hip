// The plain attention pass of the slot memory (hdcm_slot_attend_fwd, used by the backward)
// and its bf16 instantiations; the fp32 ones are in slot_attend_f32.hip.
#include "slot_kernels.h"

// ------------------------------------------------------------------ plain attention pass
extern "C" int hdcm_slot_attend_fwd(const void* base, int64_t row_stride, int64_t q_col, int64_t k_col,
                                    int64_t v_col, const void* gamma, int phi, void* ws, size_t ws_bytes,
                                    void* out, int64_t out_row_stride, int64_t out_col, const void* chain,
                                    int64_t chain_row_stride, int64_t B, int64_t L, int64_t dm, int64_t H, int64_t C,
                                    int dtype, void* stream) {
  SlotPlan pl;
  int st = slot_plan(B, L, dm, H, C, dtype, &pl);
  if (st) return st;
  HDCM_CHECK_ARG(gamma != nullptr, HDCM_EINVAL);
  HDCM_CHECK_ARG((base && out) || B == 0 || L == 0, HDCM_EINVAL);
  const int E = 16 / hdcm_elt_size(dtype);
  const int64_t ars = row_stride < 0 ? -row_stride : row_stride;
  const int64_t aors = out_row_stride < 0 ? -out_row_stride : out_row_stride;
  HDCM_CHECK_ARG(q_col >= 0 && k_col >= 0 && v_col >= 0 && out_col >= 0, HDCM_EINVAL);
  HDCM_CHECK_ARG(ars >= q_col + dm && ars >= k_col + dm && ars >= v_col + dm && aors >= out_col + dm, HDCM_EINVAL);
  HDCM_CHECK_ARG(ars < ((int64_t)1 << 31) && aors < ((int64_t)1 << 31), HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(hdcm_aligned16(base) && ars % E == 0 && q_col % E == 0 && k_col % E == 0 && v_col % E == 0 &&
                     dm % E == 0,
                 HDCM_EALIGN);
  HDCM_CHECK_ARG(((uintptr_t)out % 16) == 0 && out_col % 4 == 0 && aors % 4 == 0, HDCM_EALIGN);
  const int64_t azrs = chain_row_stride < 0 ? -chain_row_stride : chain_row_stride;
  HDCM_CHECK_ARG(!chain || (azrs >= out_col + dm && azrs < ((int64_t)1 << 31)), HDCM_EINVAL);
  HDCM_CHECK_ARG(!chain || (((uintptr_t)chain % 8) == 0 && azrs % 4 == 0), HDCM_EALIGN);
  if (B == 0 || L == 0) return HDCM_OK;
  HDCM_CHECK_ARG(ws != nullptr && ws_bytes >= slot_ws_bytes(B, H, pl), HDCM_EWORKSPACE);
  HDCM_CHECK_ARG(((uintptr_t)ws & 15u) == 0, HDCM_EALIGN);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HDCM_BF16)
    return hdcm_slot::attend_launch_bf16(base, row_stride, q_col, k_col, v_col, gamma, phi, ws, out,
                                         out_row_stride, out_col, chain, chain_row_stride, B, L, H, C, pl, s);
  return hdcm_slot::attend_launch_f32(base, row_stride, q_col, k_col, v_col, gamma, phi, ws, out,
                                      out_row_stride, out_col, chain, chain_row_stride, B, L, H, C, pl, s);
}

int hdcm_slot::attend_launch_bf16(const void* base, int64_t row_stride, int64_t q_col, int64_t k_col,
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
  HDCM_ATTEND_CASE(bf16_t, 16, true)
  HDCM_ATTEND_CASE(bf16_t, 32, true)
  HDCM_ATTEND_CASE(bf16_t, 48, true)
  HDCM_ATTEND_CASE(bf16_t, 64, true)
  HDCM_ATTEND_CASE(bf16_t, 80, true)
  HDCM_ATTEND_CASE(bf16_t, 96, true)
  HDCM_ATTEND_CASE(bf16_t, 112, true)
  HDCM_ATTEND_CASE(bf16_t, 128, true)
  HDCM_ATTEND_CASE(bf16_t, 16, false)
  HDCM_ATTEND_CASE(bf16_t, 32, false)
  HDCM_ATTEND_CASE(bf16_t, 48, false)
  HDCM_ATTEND_CASE(bf16_t, 64, false)
  HDCM_ATTEND_CASE(bf16_t, 80, false)
  HDCM_ATTEND_CASE(bf16_t, 96, false)
  HDCM_ATTEND_CASE(bf16_t, 112, false)
  HDCM_ATTEND_CASE(bf16_t, 128, false)
#undef HDCM_ATTEND_CASE
  return HDCM_EUNSUPPORTED;
}
