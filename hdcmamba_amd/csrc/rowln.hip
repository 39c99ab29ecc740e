// Row LayerNorm (fp32 statistics, optional affine) for gfx950.
//
// Replaces F.layer_norm(combined.float(), (ds+dm,)).to(dtype) at hdcmamba/model.py:382,
// which costs three full passes in PyTorch (upcast, normalise, downcast), and the
// nn.LayerNorm of HdcMamba9v3Model.norm_final (model.py:400,404).
//
// One wave owns kRows rows; it issues every 128-bit load of all its rows before the
// first reduction, so each lane keeps kRows*NG loads in flight.  Lane l owns the
// 16-byte column groups l + 64*i.  In-place use (in == out) is safe: a wave reads all
// of its rows before it writes any, and no two waves share a row.
#include "hdcm_common.h"

using namespace hdcm;

namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kRows = 4;
// Below this many rows (decode steps: one row per sequence) every row gets its own
// single-wave workgroup, so the rows spread over CUs instead of queueing in one wave.
constexpr int64_t kFewRows = 4096;

template <typename T, int NG, bool AFFINE, int kRows, int kWavesPerBlock>
__global__ __launch_bounds__(kWavesPerBlock* kWave) void rowln_kernel(
    const T* in, int64_t in_rs, T* out, int64_t out_rs, const T* __restrict__ w,
    const T* __restrict__ b, int64_t rows, int W, float eps) {
  constexpr int E = Vec<T>::N;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t r0 = ((int64_t)blockIdx.x * kWavesPerBlock + wave) * kRows;
  if (r0 >= rows) return;
  const int G = W / E;
  const float invW = 1.0f / (float)W;

  uint4 raw[kRows][NG];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int64_t row = r0 + r < rows ? r0 + r : rows - 1;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int g = lane + kWave * i;
      raw[r][i] = g < G ? ldg16(in + row * in_rs + (int64_t)g * E) : make_uint4(0, 0, 0, 0);
    }
  }

#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int64_t row = r0 + r;
    float v[NG][E];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      unpack16<T>(raw[r][i], v[i]);
#pragma unroll
      for (int e = 0; e < E; ++e) s += v[i][e];
    }
    const float mean = wave_total(s) * invW;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const bool ok = (lane + kWave * i) < G;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float c = ok ? v[i][e] - mean : 0.f;
        v[i][e] = c;
        q += c * c;
      }
    }
    const float rstd = rsqrtf(wave_total(q) * invW + eps);
    if (row < rows) {
#pragma unroll
      for (int i = 0; i < NG; ++i) {
        const int g = lane + kWave * i;
        if (g >= G) continue;
        float o[E];
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = v[i][e] * rstd;
        if (AFFINE) {
          float ww[E], bb[E];
          load16<T>(w + g * E, ww);
          load16<T>(b + g * E, bb);
#pragma unroll
          for (int e = 0; e < E; ++e) o[e] = o[e] * ww[e] + bb[e];
        }
        store16<T>(out + row * out_rs + (int64_t)g * E, o);
      }
    }
  }
}

template <typename T, int NG, int R, int WPB>
void launch_shape(const void* in, int64_t in_rs, void* out, int64_t out_rs, const void* w,
                  const void* b, int64_t rows, int64_t W, float eps, hipStream_t s) {
  const int64_t per_block = (int64_t)WPB * R;
  dim3 grid((unsigned)((rows + per_block - 1) / per_block));
  if (w)
    hipLaunchKernelGGL((rowln_kernel<T, NG, true, R, WPB>), grid, dim3(WPB * kWave), 0, s,
                       (const T*)in, in_rs, (T*)out, out_rs, (const T*)w, (const T*)b, rows, (int)W,
                       eps);
  else
    hipLaunchKernelGGL((rowln_kernel<T, NG, false, R, WPB>), grid, dim3(WPB * kWave), 0, s,
                       (const T*)in, in_rs, (T*)out, out_rs, (const T*)nullptr,
                       (const T*)nullptr, rows, (int)W, eps);
}

template <typename T, int NG>
int launch_ng(const void* in, int64_t in_rs, void* out, int64_t out_rs, const void* w,
              const void* b, int64_t rows, int64_t W, float eps, hipStream_t s) {
  if (rows < kFewRows)
    launch_shape<T, NG, 1, 1>(in, in_rs, out, out_rs, w, b, rows, W, eps, s);
  else
    launch_shape<T, NG, kRows, kWavesPerBlock>(in, in_rs, out, out_rs, w, b, rows, W, eps, s);
  return hdcm_launch_status();
}

template <typename T>
int launch(const void* in, int64_t in_rs, void* out, int64_t out_rs, const void* w,
           const void* b, int64_t rows, int64_t W, float eps, hipStream_t s) {
  const int G = (int)(W / Vec<T>::N);
  const int ng = (G + kWave - 1) / kWave;
#define HDCM_NG_CASE(n) \
  case n:               \
    return launch_ng<T, n>(in, in_rs, out, out_rs, w, b, rows, W, eps, s);
  switch (ng) {
    HDCM_NG_CASE(1)
    HDCM_NG_CASE(2)
    HDCM_NG_CASE(3)
    HDCM_NG_CASE(4)
    HDCM_NG_CASE(5)
    HDCM_NG_CASE(6)
    HDCM_NG_CASE(7)
    HDCM_NG_CASE(8)
    HDCM_NG_CASE(9)
    HDCM_NG_CASE(10)
    HDCM_NG_CASE(11)
    HDCM_NG_CASE(12)
    default:
      return HDCM_EUNSUPPORTED;
  }
#undef HDCM_NG_CASE
}

}  // namespace

extern "C" int hdcm_rowln_fwd(const void* in, int64_t in_row_stride, void* out,
                              int64_t out_row_stride, const void* w, const void* b, int64_t rows,
                              int64_t width, float eps, int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(in && out, HDCM_EINVAL);
  HDCM_CHECK_ARG((w == nullptr) == (b == nullptr), HDCM_EINVAL);
  HDCM_CHECK_ARG(rows >= 0 && width > 0, HDCM_EINVAL);
  const int E = 16 / hdcm_elt_size(dtype);
  HDCM_CHECK_ARG(width % E == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(width / E <= 12 * kWave, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(in_row_stride >= width && out_row_stride >= width, HDCM_EINVAL);
  HDCM_CHECK_ARG(in_row_stride % E == 0 && out_row_stride % E == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(hdcm_aligned16(in) && hdcm_aligned16(out), HDCM_EALIGN);
  HDCM_CHECK_ARG(!w || (hdcm_aligned16(w) && hdcm_aligned16(b)), HDCM_EALIGN);
  HDCM_CHECK_ARG(rows / (kWavesPerBlock * kRows) < ((int64_t)1 << 31), HDCM_EUNSUPPORTED);
  if (rows == 0) return HDCM_OK;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HDCM_F32)
    return launch<float>(in, in_row_stride, out, out_row_stride, w, b, rows, width, eps, s);
  return launch<bf16_t>(in, in_row_stride, out, out_row_stride, w, b, rows, width, eps, s);
}
