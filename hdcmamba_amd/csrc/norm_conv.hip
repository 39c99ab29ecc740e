// Fused LayerNorm + causal depthwise conv (width 4) forward for gfx950.
//
// Semantics follow hdcmamba/model.py:22-72: per row t, u = LN(x[t]) with biased
// variance and rsqrt(var+eps); out[t] = u[t-3]*w0 + u[t-2]*w1 + u[t-1]*w2 + u[t]*w3 + b,
// and rows t<0 contribute LN(0-row) = ln_b.
//
// Design: one 64-lane wave streams a run of R consecutive rows of one sequence.  Lane l
// owns the 16-byte column groups g = l + 64*i (i < NG), so a row costs NG 128-bit loads
// per lane and the three history rows stay in registers.  The LN affine is folded into
// the taps:  out = sum_k (w*c_k) * xhat[t-3+k] + (b*sum_k c_k + c_b), xhat = (x-mu)*rstd,
// which makes the t<0 halo exactly xhat = 0.  Raw rows are prefetched PF rows ahead so
// several 128-bit loads per lane are in flight while the current row is reduced.
//
// When half a row fills a wave (D/2 >= 64 16-byte groups, e.g. bf16 D = 1024 or 2048),
// norm_conv_split_kernel is used instead: a workgroup of two waves walks kSplitRows rows,
// wave w owning columns [w*D/2, (w+1)*D/2).  Each wave reduces its half-row on DPP lane
// moves into a scalar mean m_w and centred sum of squares M2_w; the halves are merged with
// Chan's formula (mean = (m_0+m_1)/2, M2 = M2_0 + M2_1 + (m_1-m_0)^2 * D/4) through LDS,
// one barrier per row.  Halving the columns per lane halves the registers that hold the
// folded taps and the three history rows, which raises occupancy from 2 to 4 waves per
// SIMD.  Blocks are numbered so that each XCD walks one contiguous range of rows, which
// keeps the 3-row halo of a block in the L2 that just read it as its neighbour's tail.
#include "hdcm_common.h"

using namespace hdcm;

namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kPF = 3;  // prefetch distance (rows)

template <typename T, int NG>
__device__ __forceinline__ void load_row(uint4 (&raw)[NG], const T* row, int lane, int G) {
  constexpr int E = Vec<T>::N;
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int g = lane + kWave * i;
    raw[i] = (g < G) ? ldg16(row + (int64_t)g * E) : make_uint4(0, 0, 0, 0);
  }
}

// Normalise one row in registers: xh = (x - mean) * rstd (0 on lanes past D).
template <typename T, int NG>
__device__ __forceinline__ void ln_row(const uint4 (&raw)[NG], float (&xh)[NG][Vec<T>::N], int lane,
                                       int G, float invD, float eps) {
  constexpr int E = Vec<T>::N;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    unpack16<T>(raw[i], xh[i]);
#pragma unroll
    for (int e = 0; e < E; ++e) s += xh[i][e];
  }
  const float mean = wave_sum(s) * invD;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const bool ok = (lane + kWave * i) < G;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float c = ok ? xh[i][e] - mean : 0.f;
      xh[i][e] = c;
      q += c * c;
    }
  }
  const float rstd = rsqrtf(wave_sum(q) * invD + eps);
#pragma unroll
  for (int i = 0; i < NG; ++i)
#pragma unroll
    for (int e = 0; e < E; ++e) xh[i][e] *= rstd;
}

template <typename T, int NG, int kRows>
__global__ __launch_bounds__(kWavesPerBlock* kWave) void norm_conv_kernel(
    const T* __restrict__ x, int64_t x_bs, int64_t x_rs, const T* __restrict__ ln_w,
    const T* __restrict__ ln_b, const T* __restrict__ conv_w, const T* __restrict__ conv_b,
    T* __restrict__ out, int64_t o_bs, int64_t o_rs, int L, int D, float eps) {
  constexpr int E = Vec<T>::N;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t t0 = ((int64_t)blockIdx.x * kWavesPerBlock + wave) * kRows;
  if (t0 >= L) return;
  const int G = D / E;
  const float invD = 1.0f / (float)D;
  const T* xb = x + (int64_t)blockIdx.y * x_bs;
  T* ob = out + (int64_t)blockIdx.y * o_bs;

  // Folded parameters: wc[k] = ln_w * conv_w[:,k], bt = ln_b * sum_k conv_w[:,k] + conv_b.
  float wc[4][NG][E], bt[NG][E];
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int g = lane + kWave * i;
    float w[E], bb[E], cb[E], cw[4 * E];
    if (g < G) {
      load16<T>(ln_w + g * E, w);
      load16<T>(ln_b + g * E, bb);
      load16<T>(conv_b + g * E, cb);
#pragma unroll
      for (int k = 0; k < 4; ++k) load16<T>(conv_w + (int64_t)g * E * 4 + k * E, cw + k * E);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) { w[e] = 0.f; bb[e] = 0.f; cb[e] = 0.f; }
#pragma unroll
      for (int e = 0; e < 4 * E; ++e) cw[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
      // conv_w is [D,4]: column c = g*E+e has taps cw[4e..4e+3].
      const float c0 = cw[4 * e + 0], c1 = cw[4 * e + 1], c2 = cw[4 * e + 2], c3 = cw[4 * e + 3];
      wc[0][i][e] = w[e] * c0;
      wc[1][i][e] = w[e] * c1;
      wc[2][i][e] = w[e] * c2;
      wc[3][i][e] = w[e] * c3;
      bt[i][e] = bb[e] * (c0 + c1 + c2 + c3) + cb[e];
    }
  }

  // History rows t0-3, t0-2, t0-1 (xhat = 0 before the sequence start).
  float h3[NG][E], h2[NG][E], h1[NG][E];
  {
    uint4 r3[NG], r2[NG], r1[NG];
    load_row<T, NG>(r3, xb + (t0 >= 3 ? (t0 - 3) : 0) * x_rs, lane, G);
    load_row<T, NG>(r2, xb + (t0 >= 2 ? (t0 - 2) : 0) * x_rs, lane, G);
    load_row<T, NG>(r1, xb + (t0 >= 1 ? (t0 - 1) : 0) * x_rs, lane, G);
    ln_row<T, NG>(r3, h3, lane, G, invD, eps);
    ln_row<T, NG>(r2, h2, lane, G, invD, eps);
    ln_row<T, NG>(r1, h1, lane, G, invD, eps);
    if (t0 < 3) {
#pragma unroll
      for (int i = 0; i < NG; ++i)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          if (t0 < 3) h3[i][e] = 0.f;
          if (t0 < 2) h2[i][e] = 0.f;
          if (t0 < 1) h1[i][e] = 0.f;
        }
    }
  }

  // Prefetch ring (row indices clamped in-bounds; rows >= L are never stored).
  uint4 ring[kPF][NG];
#pragma unroll
  for (int p = 0; p < kPF; ++p) {
    const int64_t t = t0 + p < L ? t0 + p : L - 1;
    load_row<T, NG>(ring[p], xb + t * x_rs, lane, G);
  }

#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    uint4 cur[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) cur[i] = ring[r % kPF][i];
    {
      const int64_t tn = t0 + r + kPF < L ? t0 + r + kPF : L - 1;
      if (r + kPF < kRows) load_row<T, NG>(ring[r % kPF], xb + tn * x_rs, lane, G);
    }
    const int64_t t = t0 + r;
    if (t >= L) break;
    float h0[NG][E];
    ln_row<T, NG>(cur, h0, lane, G, invD, eps);
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int g = lane + kWave * i;
      float o[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        o[e] = wc[0][i][e] * h3[i][e] + wc[1][i][e] * h2[i][e] + wc[2][i][e] * h1[i][e] +
               wc[3][i][e] * h0[i][e] + bt[i][e];
        h3[i][e] = h2[i][e];
        h2[i][e] = h1[i][e];
        h1[i][e] = h0[i][e];
      }
      if (g < G) store16<T>(ob + t * o_rs + (int64_t)g * E, o);
    }
  }
}


// Block index -> row-run index: XCD x (blocks are dealt to the 8 XCDs round robin) gets the
// contiguous runs [x*n/8, (x+1)*n/8), so neighbouring runs share an L2.
__device__ __forceinline__ int64_t xcd_run(int64_t b, int64_t n) {
  if (n & 7) return b;
  return (b & 7) * (n >> 3) + (b >> 3);
}

constexpr int kSplitRows = 32;
constexpr int kSplitPF = 4;

template <typename T, int NG, bool FULL>
__global__ __launch_bounds__(2 * kWave) void norm_conv_split_kernel(
    const T* __restrict__ x, int64_t x_bs, int64_t x_rs, const T* __restrict__ ln_w,
    const T* __restrict__ ln_b, const T* __restrict__ conv_w, const T* __restrict__ conv_b,
    T* __restrict__ out, int64_t o_bs, int64_t o_rs, int L, int D, float eps) {
  constexpr int E = Vec<T>::N;
  __shared__ float2 sst[2][2];  // [row parity][wave]: (half-row mean, centred sum of squares)
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  const int64_t t0 = xcd_run(blockIdx.x, gridDim.x) * kSplitRows;
  const int half = D / 2;
  const int G = half / E;  // 16-byte groups per half-row
  const float invHalf = 1.0f / (float)half, invD = 1.0f / (float)D;
  const float cross = 0.25f * (float)D;  // n_0 n_1 / n for two equal halves
  const T* xb = x + (int64_t)blockIdx.y * x_bs + w * half;
  T* ob = out + (int64_t)blockIdx.y * o_bs + w * half;

  float wc[4][NG][E], bt[NG][E];
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int g = lane + kWave * i;
    float lw[E], lb[E], cb[E], cw[4 * E];
    if (FULL || g < G) {
      const int c = w * half + g * E;
      load16<T>(ln_w + c, lw);
      load16<T>(ln_b + c, lb);
      load16<T>(conv_b + c, cb);
#pragma unroll
      for (int k = 0; k < 4; ++k) load16<T>(conv_w + (int64_t)c * 4 + k * E, cw + k * E);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) { lw[e] = 0.f; lb[e] = 0.f; cb[e] = 0.f; }
#pragma unroll
      for (int e = 0; e < 4 * E; ++e) cw[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float c0 = cw[4 * e + 0], c1 = cw[4 * e + 1], c2 = cw[4 * e + 2], c3 = cw[4 * e + 3];
      wc[0][i][e] = lw[e] * c0;
      wc[1][i][e] = lw[e] * c1;
      wc[2][i][e] = lw[e] * c2;
      wc[3][i][e] = lw[e] * c3;
      bt[i][e] = lb[e] * (c0 + c1 + c2 + c3) + cb[e];
    }
  }

  int par = 0;
  // LayerNorm of one row: every call runs in both waves (one barrier each).
  auto ln = [&](const uint4 (&raw)[NG], float (&h)[NG][E]) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      unpack16<T>(raw[i], h[i]);
#pragma unroll
      for (int e = 0; e < E; ++e) s += h[i][e];
    }
    const float mw = wave_total(s) * invHalf;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const bool ok = FULL || (lane + kWave * i) < G;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float c = ok ? h[i][e] - mw : 0.f;
        q += c * c;
      }
    }
    const float m2 = wave_total(q);
    if (lane == 0) sst[par][w] = make_float2(mw, m2);
    __syncthreads();
    const float2 o = sst[par][w ^ 1];
    par ^= 1;
    const float d = o.x - mw;
    const float mean = 0.5f * (mw + o.x);
    const float rstd = rsqrtf((m2 + o.y + d * d * cross) * invD + eps);
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int e = 0; e < E; ++e) h[i][e] = (h[i][e] - mean) * rstd;
  };

  uint4 ring[kSplitPF][NG];
#pragma unroll
  for (int p = 0; p < kSplitPF; ++p) {
    const int64_t t = t0 + p < L ? t0 + p : L - 1;
    load_row<T, NG>(ring[p], xb + t * x_rs, lane, G);
  }
  float h3[NG][E], h2[NG][E], h1[NG][E];
  {
    uint4 r3[NG], r2[NG], r1[NG];
    load_row<T, NG>(r3, xb + (t0 >= 3 ? t0 - 3 : 0) * x_rs, lane, G);
    load_row<T, NG>(r2, xb + (t0 >= 2 ? t0 - 2 : 0) * x_rs, lane, G);
    load_row<T, NG>(r1, xb + (t0 >= 1 ? t0 - 1 : 0) * x_rs, lane, G);
    ln(r3, h3);
    ln(r2, h2);
    ln(r1, h1);
    if (t0 < 3) {
#pragma unroll
      for (int i = 0; i < NG; ++i)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          if (t0 < 3) h3[i][e] = 0.f;
          if (t0 < 2) h2[i][e] = 0.f;
          if (t0 < 1) h1[i][e] = 0.f;
        }
    }
  }

#pragma unroll
  for (int r = 0; r < kSplitRows; ++r) {
    uint4 cur[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) cur[i] = ring[r % kSplitPF][i];
    if (r + kSplitPF < kSplitRows) {
      const int64_t tn = t0 + r + kSplitPF < L ? t0 + r + kSplitPF : L - 1;
      load_row<T, NG>(ring[r % kSplitPF], xb + tn * x_rs, lane, G);
    }
    // both waves run every row (the LayerNorm barrier); rows past L are not stored
    float h0[NG][E];
    ln(cur, h0);
    const int64_t t = t0 + r;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int g = lane + kWave * i;
      float o[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        o[e] = wc[0][i][e] * h3[i][e] + wc[1][i][e] * h2[i][e] + wc[2][i][e] * h1[i][e] +
               wc[3][i][e] * h0[i][e] + bt[i][e];
        h3[i][e] = h2[i][e];
        h2[i][e] = h1[i][e];
        h1[i][e] = h0[i][e];
      }
      if (t < L && (FULL || g < G)) store16<T>(ob + t * o_rs + (int64_t)g * E, o);
    }
  }
}

template <typename T, int NG>
int launch_split(const void* x, int64_t x_bs, int64_t x_rs, const void* ln_w, const void* ln_b,
                 const void* conv_w, const void* conv_b, void* out, int64_t o_bs, int64_t o_rs,
                 int64_t B, int64_t L, int64_t D, float eps, hipStream_t s) {
  dim3 grid((unsigned)((L + kSplitRows - 1) / kSplitRows), (unsigned)B);
  const bool full = (D / 2 / Vec<T>::N) == NG * kWave;
  if (full)
    hipLaunchKernelGGL((norm_conv_split_kernel<T, NG, true>), grid, dim3(2 * kWave), 0, s, (const T*)x,
                       x_bs, x_rs, (const T*)ln_w, (const T*)ln_b, (const T*)conv_w, (const T*)conv_b,
                       (T*)out, o_bs, o_rs, (int)L, (int)D, eps);
  else
    hipLaunchKernelGGL((norm_conv_split_kernel<T, NG, false>), grid, dim3(2 * kWave), 0, s, (const T*)x,
                       x_bs, x_rs, (const T*)ln_w, (const T*)ln_b, (const T*)conv_w, (const T*)conv_b,
                       (T*)out, o_bs, o_rs, (int)L, (int)D, eps);
  return hdcm_launch_status();
}

template <typename T, int NG, int kRows>
void launch_rows(const void* x, int64_t x_bs, int64_t x_rs, const void* ln_w, const void* ln_b,
                 const void* conv_w, const void* conv_b, void* out, int64_t o_bs, int64_t o_rs,
                 int64_t B, int64_t L, int64_t D, float eps, hipStream_t s) {
  const int64_t rows_per_block = (int64_t)kWavesPerBlock * kRows;
  dim3 grid((unsigned)((L + rows_per_block - 1) / rows_per_block), (unsigned)B);
  hipLaunchKernelGGL((norm_conv_kernel<T, NG, kRows>), grid, dim3(kWavesPerBlock * kWave), 0, s,
                     (const T*)x, x_bs, x_rs, (const T*)ln_w, (const T*)ln_b, (const T*)conv_w,
                     (const T*)conv_b, (T*)out, o_bs, o_rs, (int)L, (int)D, eps);
}

template <typename T, int NG>
int launch_ng(const void* x, int64_t x_bs, int64_t x_rs, const void* ln_w, const void* ln_b,
              const void* conv_w, const void* conv_b, void* out, int64_t o_bs, int64_t o_rs,
              int64_t B, int64_t L, int64_t D, float eps, hipStream_t s) {
  launch_rows<T, NG, 16>(x, x_bs, x_rs, ln_w, ln_b, conv_w, conv_b, out, o_bs, o_rs, B, L, D, eps, s);
  return hdcm_launch_status();
}

template <typename T>
int launch(const void* x, int64_t x_bs, int64_t x_rs, const void* ln_w, const void* ln_b,
           const void* conv_w, const void* conv_b, void* out, int64_t o_bs, int64_t o_rs,
           int64_t B, int64_t L, int64_t D, float eps, hipStream_t s) {
  const int G = (int)(D / Vec<T>::N);
  // two waves per row when each half-row fills a wave with whole 16-byte groups
  if (D % (2 * Vec<T>::N) == 0 && G / 2 >= kWave) {
    const int ng2 = (G / 2 + kWave - 1) / kWave;
    if (ng2 == 1)
      return launch_split<T, 1>(x, x_bs, x_rs, ln_w, ln_b, conv_w, conv_b, out, o_bs, o_rs, B, L, D, eps, s);
    if (ng2 == 2)
      return launch_split<T, 2>(x, x_bs, x_rs, ln_w, ln_b, conv_w, conv_b, out, o_bs, o_rs, B, L, D, eps, s);
  }
  const int ng = (G + kWave - 1) / kWave;
#define HDCM_NG_CASE(n) \
  case n:               \
    return launch_ng<T, n>(x, x_bs, x_rs, ln_w, ln_b, conv_w, conv_b, out, o_bs, o_rs, B, L, D, eps, s);
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

extern "C" int hdcm_norm_conv_fwd(const void* x, int64_t x_batch_stride, int64_t x_row_stride,
                                  const void* ln_w, const void* ln_b, const void* conv_w,
                                  const void* conv_b, void* out, int64_t out_batch_stride,
                                  int64_t out_row_stride, int64_t B, int64_t L, int64_t D, float eps,
                                  int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(x && ln_w && ln_b && conv_w && conv_b && out, HDCM_EINVAL);
  HDCM_CHECK_ARG(B >= 0 && L >= 0 && D > 0, HDCM_EINVAL);
  const int esz = hdcm_elt_size(dtype);
  const int E = 16 / esz;
  HDCM_CHECK_ARG(D % E == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(D / E <= 12 * kWave, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(B <= 65535 && L < (int64_t)1 << 30, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(x_row_stride >= D && out_row_stride >= D, HDCM_EINVAL);
  HDCM_CHECK_ARG(x_row_stride % E == 0 && out_row_stride % E == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(x_batch_stride % E == 0 && out_batch_stride % E == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(hdcm_aligned16(x) && hdcm_aligned16(out) && hdcm_aligned16(ln_w) &&
                     hdcm_aligned16(ln_b) && hdcm_aligned16(conv_w) && hdcm_aligned16(conv_b),
                 HDCM_EALIGN);
  if (B == 0 || L == 0) return HDCM_OK;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HDCM_F32)
    return launch<float>(x, x_batch_stride, x_row_stride, ln_w, ln_b, conv_w, conv_b, out,
                         out_batch_stride, out_row_stride, B, L, D, eps, s);
  return launch<bf16_t>(x, x_batch_stride, x_row_stride, ln_w, ln_b, conv_w, conv_b, out,
                        out_batch_stride, out_row_stride, B, L, D, eps, s);
}
