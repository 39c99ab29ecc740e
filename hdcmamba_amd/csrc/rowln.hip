// Row LayerNorm (fp32 statistics, optional affine) for gfx950.
//
// Replaces F.layer_norm(combined.float(), (ds+dm,)).to(dtype) at hdcmamba/model.py:382,
// which costs three full passes in PyTorch (upcast, normalise, downcast), and the
// nn.LayerNorm of HdcMamba9v3Model.norm_final (model.py:400,404).  rowln2_kernel applies
// two LayerNorms in one pass (the LM forward's norm_final, then the wrapper's norm_f at
// train_fineweb.py:67,94), the intermediate rounded to the activation dtype as a stored
// tensor would be, with the same per-row code: it equals two rowln_kernel passes bit for bit.
//
// One wave owns kRows rows; it issues every 128-bit load of all its rows before the
// first reduction, so each lane keeps kRows*NG loads in flight.  Lane l owns the
// 16-byte column groups l + 64*i.  In-place use (in == out) is safe: a wave reads all
// of its rows before it writes any, and no two waves share a row.
#include <type_traits>

#include "hdcm_common.h"

using namespace hdcm;

namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kRows = 4;
// rowln2_kernel (norm_final then norm_f at the LM's 32768 x 1024 rows) with 2 rows per wave:
// 23.8-23.9 against 27.0-27.5 us with 4 (35.9 with 8, 24.7-25.2 with 2 rows and 8 waves per
// workgroup), alternated twice on one box
constexpr int kRows2 = 2;
// Below this many rows (decode steps: one row per sequence) every row gets its own
// single-wave workgroup, so the rows spread over CUs instead of queueing in one wave.
constexpr int64_t kFewRows = 4096;

// LayerNorm of one row held as raw 16-byte words (lane l owns groups l + 64 i): centred
// (two-pass) variance in fp32, then the affine; the outputs in fp32, zeros past the row.
template <typename T, int NG, bool AFFINE>
__device__ __forceinline__ void ln_row(const uint4 (&raw)[NG], float (&v)[NG][Vec<T>::N], int lane, int G,
                                       float invW, float eps, const uint4 (&wr)[NG], const uint4 (&br)[NG]) {
  constexpr int E = Vec<T>::N;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    unpack16<T>(raw[i], v[i]);
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
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int g = lane + kWave * i;
#pragma unroll
    for (int e = 0; e < E; ++e) v[i][e] *= rstd;
    if (AFFINE && g < G) {
      float ww[E], bb[E];
      unpack16<T>(wr[i], ww);
      unpack16<T>(br[i], bb);
#pragma unroll
      for (int e = 0; e < E; ++e) v[i][e] = v[i][e] * ww[e] + bb[e];
    }
  }
}

// The affine's weight and bias groups of this lane, as stored (loaded with the rows, so no
// load waits behind a row's reductions).
template <typename T, int NG>
__device__ __forceinline__ void load_affine(const T* __restrict__ w, const T* __restrict__ b, int lane, int G,
                                            uint4 (&wr)[NG], uint4 (&br)[NG]) {
  constexpr int E = Vec<T>::N;
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int g = lane + kWave * i;
    wr[i] = g < G ? ldg16(w + g * E) : make_uint4(0, 0, 0, 0);
    br[i] = g < G ? ldg16(b + g * E) : make_uint4(0, 0, 0, 0);
  }
}

// kRows rows of raw words of a wave, every load issued before the first reduction.
template <typename T, int NG, int kRows>
__device__ __forceinline__ void load_rows(const T* in, int64_t in_rs, int64_t r0, int64_t rows, int lane, int G,
                                          uint4 (&raw)[kRows][NG]) {
  constexpr int E = Vec<T>::N;
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int64_t row = r0 + r < rows ? r0 + r : rows - 1;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int g = lane + kWave * i;
      raw[r][i] = g < G ? ldg16(in + row * in_rs + (int64_t)g * E) : make_uint4(0, 0, 0, 0);
    }
  }
}

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
  load_rows<T, NG, kRows>(in, in_rs, r0, rows, lane, G, raw);
  uint4 wr[NG], br[NG];
  if constexpr (AFFINE) load_affine<T, NG>(w, b, lane, G, wr, br);
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int64_t row = r0 + r;
    float v[NG][E];
    ln_row<T, NG, AFFINE>(raw[r], v, lane, G, invW, eps, wr, br);
    if (row < rows) {
#pragma unroll
      for (int i = 0; i < NG; ++i) {
        const int g = lane + kWave * i;
        if (g < G) store16<T>(out + row * out_rs + (int64_t)g * E, v[i]);
      }
    }
  }
}

// Widest row of rowln2_kernel in 16-byte groups per lane: its registers hold the rows and both
// affines (8 groups: 4096 bf16 or 2048 fp32 columns).
constexpr int kRowln2MaxNG = 8;

// out = LN2(LN1(in)) with affine (w1, b1, eps1), then (w2, b2, eps2); the intermediate is
// packed to T exactly as rowln_kernel stores it.
template <typename T, int NG, int kRows, int kWavesPerBlock>
__global__ __launch_bounds__(kWavesPerBlock* kWave) void rowln2_kernel(
    const T* in, int64_t in_rs, T* out, int64_t out_rs, const T* __restrict__ w1, const T* __restrict__ b1,
    float eps1, const T* __restrict__ w2, const T* __restrict__ b2, float eps2, int64_t rows, int W) {
  constexpr int E = Vec<T>::N;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t r0 = ((int64_t)blockIdx.x * kWavesPerBlock + wave) * kRows;
  if (r0 >= rows) return;
  const int G = W / E;
  const float invW = 1.0f / (float)W;

  uint4 raw[kRows][NG];
  load_rows<T, NG, kRows>(in, in_rs, r0, rows, lane, G, raw);
  // both affines ride with the rows (up to 8 groups per lane, kRowln2MaxNG)
  uint4 w1r[NG], b1r[NG], w2r[NG], b2r[NG];
  load_affine<T, NG>(w1, b1, lane, G, w1r, b1r);
  load_affine<T, NG>(w2, b2, lane, G, w2r, b2r);
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int64_t row = r0 + r;
    float v[NG][E];
    ln_row<T, NG, true>(raw[r], v, lane, G, invW, eps1, w1r, b1r);
    uint4 mid[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) mid[i] = (lane + kWave * i) < G ? pack16<T>(v[i]) : make_uint4(0, 0, 0, 0);
    ln_row<T, NG, true>(mid, v, lane, G, invW, eps2, w2r, b2r);
    if (row < rows) {
#pragma unroll
      for (int i = 0; i < NG; ++i) {
        const int g = lane + kWave * i;
        if (g < G) store16<T>(out + row * out_rs + (int64_t)g * E, v[i]);
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
    HDCM_LAUNCH((rowln_kernel<T, NG, true, R, WPB>), grid, dim3(WPB * kWave), 0, s,
                       (const T*)in, in_rs, (T*)out, out_rs, (const T*)w, (const T*)b, rows, (int)W,
                       eps);
  else
    HDCM_LAUNCH((rowln_kernel<T, NG, false, R, WPB>), grid, dim3(WPB * kWave), 0, s,
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

// f(std::integral_constant<int, NG>{}) for the 16-byte groups per lane (NG <= MaxNG <= 12) that
// a row of W values needs.
template <typename T, int MaxNG, typename F>
int with_ng(int64_t W, F&& f) {
  const int ng = (int)((W / Vec<T>::N + kWave - 1) / kWave);
#define HDCM_NG_CASE(n)                                                       \
  case n:                                                                     \
    if constexpr (n <= MaxNG) return f(std::integral_constant<int, n>{}); \
    return HDCM_EUNSUPPORTED;
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

template <typename T>
int launch(const void* in, int64_t in_rs, void* out, int64_t out_rs, const void* w,
           const void* b, int64_t rows, int64_t W, float eps, hipStream_t s) {
  return with_ng<T, 12>(W, [&](auto ng) { return launch_ng<T, decltype(ng)::value>(in, in_rs, out, out_rs, w, b, rows, W, eps, s); });
}

template <typename T, int NG, int R, int WPB>
void launch2_shape(const void* in, int64_t in_rs, void* out, int64_t out_rs, const void* w1, const void* b1,
                   float eps1, const void* w2, const void* b2, float eps2, int64_t rows, int64_t W, hipStream_t s) {
  const int64_t per_block = (int64_t)WPB * R;
  HDCM_LAUNCH((rowln2_kernel<T, NG, R, WPB>), dim3((unsigned)((rows + per_block - 1) / per_block)),
              dim3(WPB * kWave), 0, s, (const T*)in, in_rs, (T*)out, out_rs, (const T*)w1, (const T*)b1, eps1,
              (const T*)w2, (const T*)b2, eps2, rows, (int)W);
}

template <typename T>
int launch2(const void* in, int64_t in_rs, void* out, int64_t out_rs, const void* w1, const void* b1, float eps1,
            const void* w2, const void* b2, float eps2, int64_t rows, int64_t W, hipStream_t s) {
  return with_ng<T, kRowln2MaxNG>(W, [&](auto ng) {
    constexpr int NG = decltype(ng)::value;
    if (rows < kFewRows)
      launch2_shape<T, NG, 1, 1>(in, in_rs, out, out_rs, w1, b1, eps1, w2, b2, eps2, rows, W, s);
    else
      launch2_shape<T, NG, kRows2, kWavesPerBlock>(in, in_rs, out, out_rs, w1, b1, eps1, w2, b2, eps2, rows, W, s);
    return hdcm_launch_status();
  });
}

}  // namespace

extern "C" int hdcm_rowln_fwd(const void* in, int64_t in_row_stride, void* out,
                              int64_t out_row_stride, const void* w, const void* b, int64_t rows,
                              int64_t width, float eps, int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG((in && out) || rows == 0, HDCM_EINVAL);  // empty inputs may have no storage
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

extern "C" int hdcm_rowln2_fwd(const void* in, int64_t in_row_stride, void* out, int64_t out_row_stride,
                               const void* w1, const void* b1, float eps1, const void* w2, const void* b2,
                               float eps2, int64_t rows, int64_t width, int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG((in && out) || rows == 0, HDCM_EINVAL);
  HDCM_CHECK_ARG(w1 && b1 && w2 && b2, HDCM_EINVAL);
  HDCM_CHECK_ARG(rows >= 0 && width > 0, HDCM_EINVAL);
  const int E = 16 / hdcm_elt_size(dtype);
  HDCM_CHECK_ARG(width % E == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(width / E <= kRowln2MaxNG * kWave, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(in_row_stride >= width && out_row_stride >= width, HDCM_EINVAL);
  HDCM_CHECK_ARG(in_row_stride % E == 0 && out_row_stride % E == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(hdcm_aligned16(in) && hdcm_aligned16(out), HDCM_EALIGN);
  HDCM_CHECK_ARG(hdcm_aligned16(w1) && hdcm_aligned16(b1) && hdcm_aligned16(w2) && hdcm_aligned16(b2),
                 HDCM_EALIGN);
  HDCM_CHECK_ARG(rows / (kWavesPerBlock * kRows) < ((int64_t)1 << 31), HDCM_EUNSUPPORTED);
  if (rows == 0) return HDCM_OK;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HDCM_F32)
    return launch2<float>(in, in_row_stride, out, out_row_stride, w1, b1, eps1, w2, b2, eps2, rows, width, s);
  return launch2<bf16_t>(in, in_row_stride, out, out_row_stride, w1, b1, eps1, w2, b2, eps2, rows, width, s);
}

// ------------------------------------------------------------------------- backward
// Gradient of the row LayerNorm above (nn.LayerNorm's backward, as autograd runs it for
// the reference's norm_final / F.layer_norm at hdcmamba/model.py:382,404):
//   x^ = (x - mean) * rstd,  g = dy * w (or dy without affine)
//   dx = rstd * (g - mean(g) - x^ * mean(g * x^))
//   dw = sum over rows of dy * x^,  db = sum over rows of dy
// The statistics are recomputed from x in fp32.  Pass 1 (one wave per row, a fixed grid of
// workgroups striding over the rows) writes dx and, with affine, each workgroup's column
// sums of dy*x^ and dy; pass 2 adds those partials in a fixed order, so dw and db are
// deterministic.
namespace {

constexpr int kBwdWaves = 4;
constexpr int kBwdMaxBlocks = 1024;

int64_t bwd_blocks(int64_t rows) {
  const int64_t need = (rows + kBwdWaves - 1) / kBwdWaves;
  return need < kBwdMaxBlocks ? (need > 0 ? need : 1) : kBwdMaxBlocks;
}

template <typename T, int NG, bool AFFINE>
__global__ __launch_bounds__(kBwdWaves* kWave) void rowln_bwd_rows_kernel(
    const T* __restrict__ dy, int64_t dy_rs, const T* __restrict__ x, int64_t x_rs,
    const T* __restrict__ w, T* __restrict__ dx, int64_t dx_rs, float* __restrict__ part,
    int64_t rows, int W, float eps) {
  constexpr int E = Vec<T>::N;
  __shared__ float red[AFFINE ? 2 : 1][AFFINE ? NG * E * kWave : 1];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int G = W / E;
  const float invW = 1.0f / (float)W;
  float ww[NG][E];
  float adw[NG][E], adb[NG][E];
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int g = lane + kWave * i;
#pragma unroll
    for (int e = 0; e < E; ++e) ww[i][e] = 1.f, adw[i][e] = 0.f, adb[i][e] = 0.f;
    if (AFFINE && g < G) load16<T>(w + (int64_t)g * E, ww[i]);
  }
  const int64_t stride = (int64_t)gridDim.x * kBwdWaves;
  for (int64_t row = (int64_t)blockIdx.x * kBwdWaves + wave; row < rows; row += stride) {
    uint4 rx[NG], rd[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int g = lane + kWave * i < G ? lane + kWave * i : 0;
      rx[i] = ldg16(x + row * x_rs + (int64_t)g * E);
      rd[i] = ldg16(dy + row * dy_rs + (int64_t)g * E);
    }
    float xv[NG][E], gv[NG][E];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const bool ok = lane + kWave * i < G;
      unpack16<T>(rx[i], xv[i]);
      unpack16<T>(rd[i], gv[i]);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        if (!ok) xv[i][e] = 0.f, gv[i][e] = 0.f;
        s += xv[i][e];
      }
    }
    const float mean = wave_total(s) * invW;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const bool ok = lane + kWave * i < G;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float c = ok ? xv[i][e] - mean : 0.f;
        xv[i][e] = c;
        q += c * c;
      }
    }
    const float rstd = rsqrtf(wave_total(q) * invW + eps);
    float sg = 0.f, sgx = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float xh = xv[i][e] * rstd;  // x^ (0 past W)
        xv[i][e] = xh;
        if (AFFINE) {
          adw[i][e] += gv[i][e] * xh;
          adb[i][e] += gv[i][e];
        }
        const float g = gv[i][e] * ww[i][e];
        gv[i][e] = g;
        sg += g;
        sgx += g * xh;
      }
    const float mg = wave_total(sg) * invW, mgx = wave_total(sgx) * invW;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int g = lane + kWave * i;
      if (g >= G) continue;
      float o[E];
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = rstd * (gv[i][e] - mg - xv[i][e] * mgx);
      store16<T>(dx + row * dx_rs + (int64_t)g * E, o);
    }
  }
  if constexpr (AFFINE) {
    // this workgroup's column sums: the waves add theirs into LDS in turn (wave order,
    // deterministic), then one row of partials per workgroup
    for (int k = 0; k < kBwdWaves; ++k) {
      if (wave == k) {
#pragma unroll
        for (int i = 0; i < NG; ++i)
#pragma unroll
          for (int e = 0; e < E; ++e) {
            const int slot = (i * kWave + lane) * E + e;  // column (lane + 64 i) * E + e
            red[0][slot] = (k ? red[0][slot] : 0.f) + adw[i][e];
            red[1][slot] = (k ? red[1][slot] : 0.f) + adb[i][e];
          }
      }
      __syncthreads();
    }
    float* pw = part + (int64_t)blockIdx.x * 2 * W;
    for (int c = threadIdx.x; c < G * E; c += kBwdWaves * kWave) {
      pw[c] = red[0][c];
      pw[W + c] = red[1][c];
    }
  }
}

template <typename T, int NG>
int launch_bwd_ng(const void* dy, int64_t dy_rs, const void* x, int64_t x_rs, const void* w, void* dx,
                  int64_t dx_rs, float* dw, float* db, float* ws, int64_t rows, int W, float eps, hipStream_t s) {
  const int64_t nb = bwd_blocks(rows);
  if (w) {
    HDCM_LAUNCH((rowln_bwd_rows_kernel<T, NG, true>), dim3((unsigned)nb), dim3(kBwdWaves * kWave), 0, s,
                       (const T*)dy, dy_rs, (const T*)x, x_rs, (const T*)w, (T*)dx, dx_rs, ws, rows, W, eps);
    int st = hdcm_launch_status();
    if (st) return st;
    return hdcm_colsum(ws, 2 * (int64_t)W, (int)nb, 2 * W, 2 * W, 0, dw, W, db, s);
  } else {
    HDCM_LAUNCH((rowln_bwd_rows_kernel<T, NG, false>), dim3((unsigned)nb), dim3(kBwdWaves * kWave), 0, s,
                       (const T*)dy, dy_rs, (const T*)x, x_rs, (const T*)nullptr, (T*)dx, dx_rs, ws, rows, W, eps);
  }
  return hdcm_launch_status();
}

template <typename T>
int launch_bwd(const void* dy, int64_t dy_rs, const void* x, int64_t x_rs, const void* w, void* dx, int64_t dx_rs,
               float* dw, float* db, float* ws, int64_t rows, int W, float eps, hipStream_t s) {
  const int G = W / Vec<T>::N;
  const int ng = (G + kWave - 1) / kWave;
#define HDCM_BWD_NG(n) \
  case n:              \
    return launch_bwd_ng<T, n>(dy, dy_rs, x, x_rs, w, dx, dx_rs, dw, db, ws, rows, W, eps, s);
  switch (ng) {
    HDCM_BWD_NG(1)
    HDCM_BWD_NG(2)
    HDCM_BWD_NG(3)
    HDCM_BWD_NG(4)
    HDCM_BWD_NG(5)
    HDCM_BWD_NG(6)
    HDCM_BWD_NG(7)
    HDCM_BWD_NG(8)
    default:
      return HDCM_EUNSUPPORTED;
  }
#undef HDCM_BWD_NG
}

}  // namespace

extern "C" size_t hdcm_rowln_bwd_workspace_bytes(int64_t rows, int64_t width) {
  if (rows < 0 || width <= 0) return 0;
  return (size_t)bwd_blocks(rows) * 2 * (size_t)width * sizeof(float);
}

extern "C" int hdcm_rowln_bwd(const void* dy, int64_t dy_row_stride, const void* x, int64_t x_row_stride,
                              const void* w, void* dx, int64_t dx_row_stride, float* dw, float* db, void* ws,
                              size_t ws_bytes, int64_t rows, int64_t width, float eps, int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG((dy && x && dx) || rows == 0, HDCM_EINVAL);  // empty inputs may have no storage
  HDCM_CHECK_ARG(!w || (dw && db), HDCM_EINVAL);
  HDCM_CHECK_ARG(rows >= 0 && width > 0, HDCM_EINVAL);
  const int E = 16 / hdcm_elt_size(dtype);
  HDCM_CHECK_ARG(width % E == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(width / E <= 8 * kWave, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(dy_row_stride >= width && x_row_stride >= width && dx_row_stride >= width, HDCM_EINVAL);
  HDCM_CHECK_ARG(dy_row_stride % E == 0 && x_row_stride % E == 0 && dx_row_stride % E == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(hdcm_aligned16(dy) && hdcm_aligned16(x) && hdcm_aligned16(dx), HDCM_EALIGN);
  HDCM_CHECK_ARG(!w || hdcm_aligned16(w), HDCM_EALIGN);
  if (w) {
    HDCM_CHECK_ARG(ws != nullptr && ws_bytes >= hdcm_rowln_bwd_workspace_bytes(rows, width), HDCM_EWORKSPACE);
    HDCM_CHECK_ARG(((uintptr_t)ws & 15u) == 0, HDCM_EALIGN);
  }
  hipStream_t s = (hipStream_t)stream;
  if (rows == 0) {
    if (w)  // empty input: zero parameter gradients
      return hdcm_colsum((const float*)ws, 2 * width, 0, 2 * (int)width, 2 * (int)width, 0, dw, (int)width, db, s);
    return HDCM_OK;
  }
  if (dtype == HDCM_F32)
    return launch_bwd<float>(dy, dy_row_stride, x, x_row_stride, w, dx, dx_row_stride, dw, db, (float*)ws, rows,
                             (int)width, eps, s);
  return launch_bwd<bf16_t>(dy, dy_row_stride, x, x_row_stride, w, dx, dx_row_stride, dw, db, (float*)ws, rows,
                            (int)width, eps, s);
}
