// Slot memory + GroupNorm + gate: the forward entry points (workspace size, segment-start
// state pass, gate pass).  The kernels, their decomposition and launch plans are in
// slot_kernels.h; the plain attention pass of the backward is in slot_attend.hip.
#include "slot_kernels.h"

extern "C" size_t hdcm_slot_workspace_bytes(int64_t B, int64_t L, int64_t dm, int64_t H, int64_t C,
                                            int dtype) {
  SlotPlan pl;
  if (slot_plan(B, L, dm, H, C, dtype, &pl) != HDCM_OK) return 0;
  return slot_ws_bytes(B, H, pl);
}

extern "C" int hdcm_slot_state_fwd(const void* projs, int64_t proj_row_stride, int64_t q_col,
                                   const void* gamma, const float* S0, void* ws, size_t ws_bytes,
                                   int64_t B, int64_t L, int64_t dm, int64_t H, int64_t C,
                                   int dtype, void* stream) {
  SlotPlan pl;
  int st = slot_plan(B, L, dm, H, C, dtype, &pl);
  if (st) return st;
  st = check_projs(projs, proj_row_stride, q_col, dm, dtype, B == 0 || L == 0);
  if (st) return st;
  HDCM_CHECK_ARG(gamma != nullptr, HDCM_EINVAL);
  if (B == 0 || L == 0) return HDCM_OK;
  HDCM_CHECK_ARG(ws != nullptr && ws_bytes >= slot_ws_bytes(B, H, pl), HDCM_EWORKSPACE);
  HDCM_CHECK_ARG(((uintptr_t)ws & 15u) == 0, HDCM_EALIGN);
  hipStream_t s = (hipStream_t)stream;
#define HDCM_STATE_CASE(TT, HDV)                                                                  \
  if (pl.HD == HDV)                                                                              \
    return launch_state<TT, HDV, true>(projs, proj_row_stride, q_col + dm, dm, gamma, S0, ws, B, L, H, pl, s);
  if (dtype == HDCM_BF16) {
    HDCM_STATE_CASE(bf16_t, 16)
    HDCM_STATE_CASE(bf16_t, 32)
    HDCM_STATE_CASE(bf16_t, 48)
    HDCM_STATE_CASE(bf16_t, 64)
    HDCM_STATE_CASE(bf16_t, 80)
    HDCM_STATE_CASE(bf16_t, 96)
    HDCM_STATE_CASE(bf16_t, 112)
    HDCM_STATE_CASE(bf16_t, 128)
  } else {
    HDCM_STATE_CASE(float, 16)
    HDCM_STATE_CASE(float, 32)
    HDCM_STATE_CASE(float, 48)
    HDCM_STATE_CASE(float, 64)
    HDCM_STATE_CASE(float, 80)
    HDCM_STATE_CASE(float, 96)
    HDCM_STATE_CASE(float, 112)
    HDCM_STATE_CASE(float, 128)
  }
#undef HDCM_STATE_CASE
  return HDCM_EUNSUPPORTED;
}

extern "C" int hdcm_slot_gate_fwd(const void* projs, int64_t proj_row_stride, int64_t q_col,
                                  const void* gamma, const void* gn_w, const void* gn_b,
                                  float gn_eps, const void* ws, size_t ws_bytes, void* out,
                                  int64_t out_row_stride, int64_t out_col, float* S_final,
                                  float* row_stats, int64_t stats_part_stride, int64_t B, int64_t L,
                                  int64_t dm, int64_t H, int64_t C, int dtype, void* stream) {
  SlotPlan pl;
  int st = slot_plan(B, L, dm, H, C, dtype, &pl);
  if (st) return st;
  st = check_projs(projs, proj_row_stride, q_col, dm, dtype, B == 0 || L == 0);
  if (st) return st;
  HDCM_CHECK_ARG(gamma && gn_w && gn_b && (out || B == 0 || L == 0), HDCM_EINVAL);
  const int esz = hdcm_elt_size(dtype);
  HDCM_CHECK_ARG(out_col >= 0 && out_row_stride >= out_col + dm, HDCM_EINVAL);
  // Output runs of 4 elements must be naturally aligned (8 bytes bf16, 16 bytes fp32).
  HDCM_CHECK_ARG(((uintptr_t)out % (4 * esz)) == 0 && out_col % 4 == 0 && out_row_stride % 4 == 0,
                 HDCM_EALIGN);
  // row_stats: one (sum, sum of squares) pair per head and row, head-major
  HDCM_CHECK_ARG(!row_stats || stats_part_stride >= B * L, HDCM_EINVAL);
  HDCM_CHECK_ARG(((uintptr_t)row_stats & 7u) == 0, HDCM_EALIGN);
  if (B == 0 || L == 0) return HDCM_OK;
  HDCM_CHECK_ARG(ws != nullptr && ws_bytes >= slot_ws_bytes(B, H, pl), HDCM_EWORKSPACE);
  HDCM_CHECK_ARG(((uintptr_t)ws & 15u) == 0, HDCM_EALIGN);
  hipStream_t s = (hipStream_t)stream;
#define HDCM_GATE_CASE(TT, HDV)                                                                 \
  if (pl.HD == HDV)                                                                            \
    return launch_gate<TT, HDV, true, true>(projs, proj_row_stride, q_col, dm, 2 * dm, 3 * dm, gamma, gn_w,  \
                                            gn_b, gn_eps, ws, out, out_row_stride, out_col, S_final, row_stats, \
                                            stats_part_stride, B, L, H, C, pl, s);
  if (dtype == HDCM_BF16) {
    HDCM_GATE_CASE(bf16_t, 16)
    HDCM_GATE_CASE(bf16_t, 32)
    HDCM_GATE_CASE(bf16_t, 48)
    HDCM_GATE_CASE(bf16_t, 64)
    HDCM_GATE_CASE(bf16_t, 80)
    HDCM_GATE_CASE(bf16_t, 96)
    HDCM_GATE_CASE(bf16_t, 112)
    HDCM_GATE_CASE(bf16_t, 128)
  } else {
    HDCM_GATE_CASE(float, 16)
    HDCM_GATE_CASE(float, 32)
    HDCM_GATE_CASE(float, 48)
    HDCM_GATE_CASE(float, 64)
    HDCM_GATE_CASE(float, 80)
    HDCM_GATE_CASE(float, 96)
    HDCM_GATE_CASE(float, 112)
    HDCM_GATE_CASE(float, 128)
  }
#undef HDCM_GATE_CASE
  return HDCM_EUNSUPPORTED;
}
