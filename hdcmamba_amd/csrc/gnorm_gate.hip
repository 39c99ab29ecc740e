// GroupNorm + sigmoid gate as a pass of its own, for slot heads wider than the fused gate
// pass holds (hdcmamba/model.py:274-293, intended form): per token and head h over the head's
// hd values,  out = ((y - mean) * rstd * gn_w + gn_b) * sigmoid(gate),  y = y1 + y2', where
// y2' is y2 with the two halves of every head exchanged (column h*hd + j of y2' is column
// h*hd + (j + hd/2) mod hd of y2).  A head of 2*hb columns runs its slot recurrence as two
// sub-heads of hb (the key-block x value-block terms with equal blocks in y1, the crossed ones
// in y2, whose value blocks were exchanged before the pass), so y1 + y2' is the head's output.
// One wave per (token, head); lane i holds columns i, i+64, ...; statistics in fp32.
#include "hdcm_common.h"

using namespace hdcm;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxHeadDim = 512;

template <typename T>
__global__ __launch_bounds__(kThreads) void gnorm_gate_fwd_kernel(
    const T* __restrict__ y1, int64_t y1_rs, const T* __restrict__ y2, int64_t y2_rs, const T* __restrict__ gate,
    int64_t g_rs, const T* __restrict__ gn_w, const T* __restrict__ gn_b, float eps, T* __restrict__ out,
    int64_t o_rs, float* __restrict__ row_stats, int64_t stats_ps, int64_t rows, int hd, int H) {
  constexpr int NV = kMaxHeadDim / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t pair = (int64_t)blockIdx.x * kWaves + threadIdx.x / kWave;  // (row, head)
  if (pair >= rows * H) return;
  const int64_t r = pair / H;
  const int h = (int)(pair - r * H);
  const int half = hd / 2;
  const int c0 = h * hd;
  float y[NV], gt[NV];
  // every load first: y1, y2 (halves exchanged), the gate
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int j = lane + kWave * k;
    y[k] = 0.f;
    gt[k] = 0.f;
    if (j < hd) {
      y[k] = to_f<T>(y1[r * y1_rs + c0 + j]);
      if (y2 != nullptr) y[k] += to_f<T>(y2[r * y2_rs + c0 + (j < half ? j + half : j - half)]);
      gt[k] = to_f<T>(gate[r * g_rs + c0 + j]);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) s += y[k];
  const float mean = wave_sum(s) / (float)hd;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int j = lane + kWave * k;
    const float d = j < hd ? y[k] - mean : 0.f;
    q += d * d;
  }
  const float rstd = rsqrtf(wave_sum(q) / (float)hd + eps);
  float s1 = 0.f, s2 = 0.f;  // the stored values' sum and sum of squares (row statistics)
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int j = lane + kWave * k;
    if (j < hd) {
      const float yn = (y[k] - mean) * rstd * to_f<T>(gn_w[c0 + j]) + to_f<T>(gn_b[c0 + j]);
      const T o = from_f<T>(yn * frcp(1.0f + fexp(-gt[k])));
      out[r * o_rs + c0 + j] = o;
      const float v = to_f<T>(o);
      s1 += v;
      s2 += v * v;
    }
  }
  if (row_stats != nullptr) {
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    if (lane == 0) *reinterpret_cast<float2*>(row_stats + 2 * (h * stats_ps + r)) = make_float2(s1, s2);
  }
}

}  // namespace

extern "C" int hdcm_gnorm_gate_fwd(const void* y1, int64_t y1_row_stride, const void* y2, int64_t y2_row_stride,
                                   const void* gate, int64_t gate_row_stride, const void* gn_w, const void* gn_b,
                                   float gn_eps, void* out, int64_t out_row_stride, float* row_stats,
                                   int64_t stats_part_stride, int64_t rows, int64_t dm, int64_t H, int dtype,
                                   void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(rows >= 0 && dm > 0 && H > 0 && dm % H == 0, HDCM_EINVAL);
  HDCM_CHECK_ARG(gn_w && gn_b && ((y1 && gate && out) || rows == 0), HDCM_EINVAL);
  HDCM_CHECK_ARG(y1_row_stride >= dm && gate_row_stride >= dm && out_row_stride >= dm &&
                     (!y2 || y2_row_stride >= dm),
                 HDCM_EINVAL);
  const int64_t hd = dm / H;
  HDCM_CHECK_ARG(hd <= kMaxHeadDim && (!y2 || hd % 2 == 0), HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(!row_stats || stats_part_stride >= rows, HDCM_EINVAL);
  HDCM_CHECK_ARG(rows * H < ((int64_t)1 << 40), HDCM_EUNSUPPORTED);
  if (rows == 0) return HDCM_OK;
  const int64_t blocks = (rows * H + kWaves - 1) / kWaves;
  HDCM_CHECK_ARG(blocks < ((int64_t)1 << 31), HDCM_EUNSUPPORTED);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HDCM_F32)
    HDCM_LAUNCH((gnorm_gate_fwd_kernel<float>), dim3((unsigned)blocks), dim3(kThreads), 0, s, (const float*)y1,
                y1_row_stride, (const float*)y2, y2_row_stride, (const float*)gate, gate_row_stride,
                (const float*)gn_w, (const float*)gn_b, gn_eps, (float*)out, out_row_stride, row_stats,
                stats_part_stride, rows, (int)hd, (int)H);
  else
    HDCM_LAUNCH((gnorm_gate_fwd_kernel<bf16_t>), dim3((unsigned)blocks), dim3(kThreads), 0, s, (const bf16_t*)y1,
                y1_row_stride, (const bf16_t*)y2, y2_row_stride, (const bf16_t*)gate, gate_row_stride,
                (const bf16_t*)gn_w, (const bf16_t*)gn_b, gn_eps, (bf16_t*)out, out_row_stride, row_stats,
                stats_part_stride, rows, (int)hd, (int)H);
  return hdcm_launch_status();
}
