// Backward of the fused LayerNorm + causal depthwise conv (width 4) for gfx950.
//
// Forward (norm_conv.hip; hdcmamba/model.py:22-72): xh[t] = (x[t] - mu_t) * r_t,
// u[t] = xh[t] * g + b for t >= 0 and u[t] = b for t < 0 (the LayerNorm of a zero row),
// out[t] = sum_k w_k u[t-3+k] + cb.  With go = dL/dout this computes the exact gradients
// of that forward (hdcmamba/model.py:74-166 is the reference's backward, which drops the
// b terms of dw and db and works from bf16-rounded statistics; see the oracle):
//   gu[t]  = sum_k w_k go[t+3-k]                     (t >= 0; go past L is 0)
//   dx[t]  = r_t (gh - mean(gh) - xh[t] mean(gh xh[t])),  gh = gu[t] g
//   dg     = sum_{t>=0} gu[t] xh[t]
//   db     = sum_{t>=0} gu[t] + sum_{t, k: t-3+k<0} w_k go[t]
//   dcb    = sum_t go[t]
//   dw_k   = sum_t go[t] u[t-3+k]
//
// norm_conv_bwd_rows_kernel: one wave per 16-row run, lanes own 16-byte column groups (as
// the forward); a ring holds go[t..t+3]; writes dx and the row statistics (mu_t, r_t).  Rows
// wider than 8 groups per lane (fp32) or 4 (bf16), i.e. D > 2048, take the same kernel with
// the four waves of a workgroup sharing each row (WPR = 4: 256 column lanes, row sums
// finished across the waves in LDS), up to the forward's 768 groups per row.
// norm_conv_bwd_cols_kernel: thread = one 16-byte column group x one chunk of rows; walks
// the chunk keeping go[t..t+3] and u[t-3..t] in registers, with the next four rows' loads in
// flight while the current four are summed, and writes the seven column sums of its chunk.  colsum_kernel sums the chunks in a fixed order (the result does not depend
// on scheduling).
#include "hdcm_common.h"

using namespace hdcm;

namespace {

constexpr int kRowsWPB = 4;   // waves per workgroup, rows kernel
constexpr int kRunRows = 16;  // rows per wave, rows kernel
constexpr int kChunk = 64;    // rows per chunk, column kernel
constexpr int kStep = 4;      // rows loaded ahead, column kernel
constexpr int kColThreads = 64;

template <typename T, int NG, int CW = kWave>
__device__ __forceinline__ void ld_row(float (&v)[NG][Vec<T>::N], const T* row, int lane, int G, bool valid) {
  constexpr int E = Vec<T>::N;
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int g = lane + CW * i;
    if (valid && g < G) {
      load16<T>(row + (int64_t)g * E, v[i]);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) v[i][e] = 0.f;
    }
  }
}

// WPR waves per row: 1 (each wave its own run of rows) or kRowsWPB (the workgroup's waves
// share one run, thread = column lane).
template <typename T, int NG, int WPR>
__global__ __launch_bounds__(kRowsWPB* kWave) void norm_conv_bwd_rows_kernel(
    const T* __restrict__ go, int64_t g_bs, int64_t g_rs, const T* __restrict__ x, int64_t x_bs, int64_t x_rs,
    const T* __restrict__ ln_w, const T* __restrict__ conv_w, T* __restrict__ dx, int64_t d_bs, int64_t d_rs,
    float2* __restrict__ stats, int L, int D, float eps) {
  static_assert(WPR == 1 || WPR == kRowsWPB, "a row is one wave or the whole workgroup");
  constexpr int E = Vec<T>::N;
  constexpr int CW = WPR * kWave;  // column lanes of a row
  __shared__ float red[2][kRowsWPB][2];
  const int wave = threadIdx.x / kWave;
  const int lane = WPR == 1 ? (int)(threadIdx.x & (kWave - 1)) : (int)threadIdx.x;  // column lane
  const int64_t t0 = (WPR == 1 ? (int64_t)blockIdx.x * kRowsWPB + wave : (int64_t)blockIdx.x) * kRunRows;
  if (t0 >= L) return;  // (WPR > 1: the same for every wave of the workgroup)
  // Row totals of one or two values: within the wave, then (WPR > 1) across the waves through
  // LDS.  Two buffers used in turn: a buffer is written again only two reductions later, after
  // the barrier of the reduction between, which every thread passes after reading it.
  int parity = 0;
  auto row_total2 = [&](float& a, float& c) {
    a = wave_total(a);
    c = wave_total(c);
    if constexpr (WPR > 1) {
      if ((threadIdx.x & (kWave - 1)) == 0) {
        red[parity][wave][0] = a;
        red[parity][wave][1] = c;
      }
      __syncthreads();
      a = c = 0.f;
#pragma unroll
      for (int k = 0; k < WPR; ++k) {
        a += red[parity][k][0];
        c += red[parity][k][1];
      }
      parity ^= 1;
    }
  };
  auto row_total = [&](float a) {
    float c = 0.f;
    row_total2(a, c);
    return a;
  };
  const int b = blockIdx.y;
  const int G = D / E;
  const float invD = 1.0f / (float)D;
  const T* gb = go + (int64_t)b * g_bs;
  const T* xb = x + (int64_t)b * x_bs;
  T* db = dx + (int64_t)b * d_bs;

  float gw[NG][E], cw[4][NG][E];
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int g = lane + CW * i;
    float c4[4 * E];
    if (g < G) {
      load16<T>(ln_w + g * E, gw[i]);
#pragma unroll
      for (int k = 0; k < 4; ++k) load16<T>(conv_w + (int64_t)g * E * 4 + k * E, c4 + k * E);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) gw[i][e] = 0.f;
#pragma unroll
      for (int e = 0; e < 4 * E; ++e) c4[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < E; ++e)
#pragma unroll
      for (int k = 0; k < 4; ++k) cw[k][i][e] = c4[4 * e + k];
  }

  // go ring: r0 = go[t], r1 = go[t+1], r2 = go[t+2]; go[t+3] is loaded each row
  float r0[NG][E], r1[NG][E], r2[NG][E];
  ld_row<T, NG, CW>(r0, gb + t0 * g_rs, lane, G, true);
  ld_row<T, NG, CW>(r1, gb + (t0 + 1) * g_rs, lane, G, t0 + 1 < L);
  ld_row<T, NG, CW>(r2, gb + (t0 + 2) * g_rs, lane, G, t0 + 2 < L);

#pragma unroll 1
  for (int r = 0; r < kRunRows; ++r) {
    const int64_t t = t0 + r;
    if (t >= L) break;
    float r3[NG][E], xv[NG][E];
    ld_row<T, NG, CW>(r3, gb + (t + 3) * g_rs, lane, G, t + 3 < L);
    ld_row<T, NG, CW>(xv, xb + t * x_rs, lane, G, true);
    // row statistics of x[t]
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int e = 0; e < E; ++e) s += xv[i][e];
    const float mean = row_total(s) * invD;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const bool ok = (lane + CW * i) < G;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float c = ok ? xv[i][e] - mean : 0.f;
        xv[i][e] = c;
        q += c * c;
      }
    }
    const float rstd = rsqrtf(row_total(q) * invD + eps);
    // gh = (sum_k w_k go[t+3-k]) * g, and the two row sums of the LayerNorm backward
    float gh[NG][E];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float gu = cw[3][i][e] * r0[i][e] + cw[2][i][e] * r1[i][e] + cw[1][i][e] * r2[i][e] +
                         cw[0][i][e] * r3[i][e];
        gh[i][e] = gu * gw[i][e];
        xv[i][e] *= rstd;  // xh
        s1 += gh[i][e];
        s2 += gh[i][e] * xv[i][e];
      }
    row_total2(s1, s2);
    const float m1 = s1 * invD, m2 = s2 * invD;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int g = lane + CW * i;
      float o[E];
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = rstd * (gh[i][e] - m1 - xv[i][e] * m2);
      if (g < G) store16<T>(db + t * d_rs + (int64_t)g * E, o);
    }
    if (lane == 0) stats[(int64_t)b * L + t] = make_float2(mean, rstd);
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        r0[i][e] = r1[i][e];
        r1[i][e] = r2[i][e];
        r2[i][e] = r3[i][e];
      }
  }
}

template <typename T>
__global__ __launch_bounds__(kColThreads) void norm_conv_bwd_cols_kernel(
    const T* __restrict__ go, int64_t g_bs, int64_t g_rs, const T* __restrict__ x, int64_t x_bs, int64_t x_rs,
    const T* __restrict__ ln_w, const T* __restrict__ ln_b, const T* __restrict__ conv_w,
    const float2* __restrict__ stats, float* __restrict__ part, int L, int D, int nchunk) {
  constexpr int E = Vec<T>::N;
  const int G = D / E;
  const int gi = blockIdx.x * kColThreads + threadIdx.x;
  const int chunk = blockIdx.y, b = blockIdx.z;
  if (gi >= G) return;
  const int c0 = gi * E;
  const int t0 = chunk * kChunk;
  const int t1 = min(L, t0 + kChunk);
  const T* gb = go + (int64_t)b * g_bs + c0;
  const T* xb = x + (int64_t)b * x_bs + c0;
  const float2* st = stats + (int64_t)b * L;

  float gw[E], gbias[E], cw[4][E];
  {
    float c4[4 * E];
    load16<T>(ln_w + c0, gw);
    load16<T>(ln_b + c0, gbias);
#pragma unroll
    for (int k = 0; k < 4; ++k) load16<T>(conv_w + (int64_t)c0 * 4 + k * E, c4 + k * E);
#pragma unroll
    for (int e = 0; e < E; ++e)
#pragma unroll
      for (int k = 0; k < 4; ++k) cw[k][e] = c4[4 * e + k];
  }
  auto u_of = [&](int t, float (&u)[E]) {  // u[t] = xh[t] g + b, or b before the sequence start
    if (t < 0) {
#pragma unroll
      for (int e = 0; e < E; ++e) u[e] = gbias[e];
      return;
    }
    float xv[E];
    load16<T>(xb + (int64_t)t * x_rs, xv);
    const float2 sv = st[t];
#pragma unroll
    for (int e = 0; e < E; ++e) u[e] = (xv[e] - sv.x) * sv.y * gw[e] + gbias[e];
  };
  auto go_of = [&](int t, float (&g)[E]) {
    if (t < L) {
      load16<T>(gb + (int64_t)t * g_rs, g);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) g[e] = 0.f;
    }
  };
  // raw 16-byte groups of kStep rows: go[t+3+i], x[t+i] and (mu, r) of row t+i
  auto fetch = [&](int t, uint4 (&rg)[kStep], uint4 (&rx)[kStep], float (&rm)[kStep], float (&rr)[kStep]) {
#pragma unroll
    for (int i = 0; i < kStep; ++i) {
      rg[i] = rx[i] = make_uint4(0, 0, 0, 0);
      rm[i] = rr[i] = 0.f;
      if (t + 3 + i < L) rg[i] = ldg16(gb + (int64_t)(t + 3 + i) * g_rs);
      if (t + i < t1) {
        rx[i] = ldg16(xb + (int64_t)(t + i) * x_rs);
        const float2 sv = st[t + i];
        rm[i] = sv.x;
        rr[i] = sv.y;
      }
    }
  };

  float acc[7][E];
#pragma unroll
  for (int j = 0; j < 7; ++j)
#pragma unroll
    for (int e = 0; e < E; ++e) acc[j][e] = 0.f;
  float u3[E], u2[E], u1[E];  // u[t-3], u[t-2], u[t-1]
  u_of(t0 - 3, u3);
  u_of(t0 - 2, u2);
  u_of(t0 - 1, u1);
  float g0[E], g1[E], g2[E];  // go[t], go[t+1], go[t+2]
  go_of(t0, g0);
  go_of(t0 + 1, g1);
  go_of(t0 + 2, g2);
  uint4 ng[kStep], nx[kStep];
  float nm[kStep], nr[kStep];
  fetch(t0, ng, nx, nm, nr);
#pragma unroll 1
  for (int tb = t0; tb < t1; tb += kStep) {
    uint4 cg[kStep], cx[kStep];
    float cm[kStep], cr[kStep];
#pragma unroll
    for (int i = 0; i < kStep; ++i) {
      cg[i] = ng[i];
      cx[i] = nx[i];
      cm[i] = nm[i];
      cr[i] = nr[i];
    }
    if (tb + kStep < t1) fetch(tb + kStep, ng, nx, nm, nr);  // next rows in flight while these are summed
#pragma unroll
    for (int i = 0; i < kStep; ++i) {
      const int t = tb + i;
      if (t >= t1) continue;  // uniform: rows past the chunk
      float g3[E], xh[E];
      unpack16<T>(cg[i], g3);
      unpack16<T>(cx[i], xh);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        xh[e] = (xh[e] - cm[i]) * cr[i];
        const float u0 = xh[e] * gw[e] + gbias[e];
        const float gu = cw[3][e] * g0[e] + cw[2][e] * g1[e] + cw[1][e] * g2[e] + cw[0][e] * g3[e];
        acc[0][e] += gu * xh[e];      // dg
        acc[1][e] += gu;              // db (rows t >= 0)
        acc[2][e] += g0[e];           // dcb
        acc[3][e] += g0[e] * u3[e];   // dw0
        acc[4][e] += g0[e] * u2[e];   // dw1
        acc[5][e] += g0[e] * u1[e];   // dw2
        acc[6][e] += g0[e] * u0;      // dw3
        u3[e] = u2[e];
        u2[e] = u1[e];
        u1[e] = u0;
      }
      // the b of the rows before the sequence start feeds out[t] for t < 3
      if (t < 3) {
#pragma unroll
        for (int e = 0; e < E; ++e)
#pragma unroll
          for (int k = 0; k < 3; ++k)
            if (t - 3 + k < 0) acc[1][e] += cw[k][e] * g0[e];
      }
#pragma unroll
      for (int e = 0; e < E; ++e) {
        g0[e] = g1[e];
        g1[e] = g2[e];
        g2[e] = g3[e];
      }
    }
  }
  // part row: [dg (D) | db (D) | dcb (D) | dw (D x 4, the layout of conv_w)]
  float* pp = part + ((int64_t)b * nchunk + chunk) * 7 * D;
#pragma unroll
  for (int j = 0; j < 3; ++j)
#pragma unroll
    for (int e = 0; e < E; ++e) pp[(int64_t)j * D + c0 + e] = acc[j][e];
#pragma unroll
  for (int e = 0; e < E; ++e)
#pragma unroll
    for (int k = 0; k < 4; ++k) pp[3 * (int64_t)D + (int64_t)(c0 + e) * 4 + k] = acc[3 + k][e];
}

// Sum the part rows (nparts of them) into the four parameter gradients.
int reduce_parts(const float* part, int nparts, int64_t D, float* d_ln_w, float* d_ln_b, float* d_conv_w,
                 float* d_conv_b, hipStream_t s) {
  const int64_t ks = 7 * D;
  int st = hdcm_colsum(part, ks, nparts, 2 * (int)D, 2 * (int)D, 0, d_ln_w, (int)D, d_ln_b, s);
  if (!st) st = hdcm_colsum(part ? part + 2 * D : part, ks, nparts, (int)D, (int)D, 0, d_conv_b, (int)D, nullptr, s);
  if (!st) st = hdcm_colsum(part ? part + 3 * D : part, ks, nparts, 4 * (int)D, 4 * (int)D, 0, d_conv_w, 4 * (int)D,
                            nullptr, s);
  return st;
}

int64_t chunks_of(int64_t L) { return (L + kChunk - 1) / kChunk; }

template <typename T>
int launch_bwd(const void* go, int64_t g_bs, int64_t g_rs, const void* x, int64_t x_bs, int64_t x_rs,
               const void* ln_w, const void* ln_b, const void* conv_w, void* dx, int64_t d_bs, int64_t d_rs,
               float* d_ln_w, float* d_ln_b, float* d_conv_w, float* d_conv_b, void* ws, int64_t B, int64_t L,
               int64_t D, float eps, hipStream_t s) {
  constexpr int E = Vec<T>::N;
  const int G = (int)(D / E);
  const int ng = (G + kWave - 1) / kWave;
  float2* stats = (float2*)ws;
  float* part = (float*)((char*)ws + ((B * L * sizeof(float2) + 255) / 256) * 256);
  const int64_t nchunk = chunks_of(L);
  const dim3 rgrid((unsigned)((L + kRowsWPB * kRunRows - 1) / (kRowsWPB * kRunRows)), (unsigned)B);
  const dim3 rgrid_wide((unsigned)((L + kRunRows - 1) / kRunRows), (unsigned)B);  // a run per workgroup
#define HDCM_BWD_ROWS(N)                                                                                         \
  if (ng <= N)                                                                                                   \
    HDCM_LAUNCH((norm_conv_bwd_rows_kernel<T, N, 1>), rgrid, dim3(kRowsWPB * kWave), 0, s, (const T*)go,   \
                       g_bs, g_rs, (const T*)x, x_bs, x_rs, (const T*)ln_w, (const T*)conv_w, (T*)dx, d_bs, d_rs, \
                       stats, (int)L, (int)D, eps);
  // up to 4 groups per lane: one instance per count; fp32 rows of 1028 to 2048 columns (5 to
  // 8 groups) share an 8-group instance whose lanes past the row idle (256 VGPRs + 108 AGPRs,
  // no spills; bf16 rows up to 2048 columns fit in 4 groups); wider rows (up to 768 groups:
  // bf16 6144, fp32 3072 columns) spread over the 256 threads of a workgroup, 3 groups each
  constexpr int kWideGroups = 3;
  bool launched = true;
  HDCM_BWD_ROWS(1)
  else HDCM_BWD_ROWS(2) else HDCM_BWD_ROWS(3) else HDCM_BWD_ROWS(4) else launched = false;
  if constexpr (sizeof(T) == 4) {
    if (!launched && ng <= 8) {
      HDCM_BWD_ROWS(8)
      launched = true;
    }
  }
  if (!launched && G <= kWideGroups * kRowsWPB * kWave) {
    HDCM_LAUNCH((norm_conv_bwd_rows_kernel<T, kWideGroups, kRowsWPB>), rgrid_wide, dim3(kRowsWPB * kWave), 0, s,
                (const T*)go, g_bs, g_rs, (const T*)x, x_bs, x_rs, (const T*)ln_w, (const T*)conv_w, (T*)dx, d_bs,
                d_rs, stats, (int)L, (int)D, eps);
    launched = true;
  }
  if (!launched) return HDCM_EUNSUPPORTED;
#undef HDCM_BWD_ROWS
  int st = hdcm_launch_status();
  if (st) return st;
  const dim3 cgrid((unsigned)((G + kColThreads - 1) / kColThreads), (unsigned)nchunk, (unsigned)B);
  HDCM_LAUNCH((norm_conv_bwd_cols_kernel<T>), cgrid, dim3(kColThreads), 0, s, (const T*)go, g_bs, g_rs,
                     (const T*)x, x_bs, x_rs, (const T*)ln_w, (const T*)ln_b, (const T*)conv_w,
                     (const float2*)stats, part, (int)L, (int)D, (int)nchunk);
  st = hdcm_launch_status();
  if (st) return st;
  return reduce_parts(part, (int)(B * nchunk), D, d_ln_w, d_ln_b, d_conv_w, d_conv_b, s);
}

}  // namespace

extern "C" size_t hdcm_norm_conv_bwd_workspace_bytes(int64_t B, int64_t L, int64_t D) {
  if (B <= 0 || L <= 0 || D <= 0) return 0;
  return (size_t)((B * L * sizeof(float2) + 255) / 256) * 256 + (size_t)B * chunks_of(L) * 7 * D * sizeof(float);
}

extern "C" int hdcm_norm_conv_bwd(const void* grad_out, int64_t g_batch_stride, int64_t g_row_stride,
                                  const void* x, int64_t x_batch_stride, int64_t x_row_stride, const void* ln_w,
                                  const void* ln_b, const void* conv_w, void* dx, int64_t dx_batch_stride,
                                  int64_t dx_row_stride, float* d_ln_w, float* d_ln_b, float* d_conv_w,
                                  float* d_conv_b, void* ws, size_t ws_bytes, int64_t B, int64_t L, int64_t D,
                                  float eps, int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(ln_w && ln_b && conv_w && d_ln_w && d_ln_b && d_conv_w && d_conv_b &&
                     ((grad_out && x && dx) || B == 0 || L == 0),
                 HDCM_EINVAL);
  HDCM_CHECK_ARG(B >= 0 && L >= 0 && D > 0, HDCM_EINVAL);
  const int E = 16 / hdcm_elt_size(dtype);
  HDCM_CHECK_ARG(D % E == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(D / (16 / hdcm_elt_size(dtype)) <= 768, HDCM_EUNSUPPORTED);  // bf16 6144, fp32 3072 (the forward's)
  HDCM_CHECK_ARG(B <= 65535 && L < (int64_t)1 << 30 && (L + kChunk - 1) / kChunk <= 65535, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(hdcm_aligned16(ln_w) && hdcm_aligned16(ln_b) && hdcm_aligned16(conv_w), HDCM_EALIGN);
  if (B == 0 || L == 0)  // no rows (strides unused): the parameter gradients are zero
    return reduce_parts(nullptr, 0, D, d_ln_w, d_ln_b, d_conv_w, d_conv_b, (hipStream_t)stream);
  HDCM_CHECK_ARG(g_row_stride >= D && x_row_stride >= D && dx_row_stride >= D, HDCM_EINVAL);
  HDCM_CHECK_ARG(g_row_stride % E == 0 && x_row_stride % E == 0 && dx_row_stride % E == 0 && g_batch_stride % E == 0 &&
                     x_batch_stride % E == 0 && dx_batch_stride % E == 0,
                 HDCM_EALIGN);
  HDCM_CHECK_ARG(hdcm_aligned16(grad_out) && hdcm_aligned16(x) && hdcm_aligned16(dx) && hdcm_aligned16(ln_w) &&
                     hdcm_aligned16(ln_b) && hdcm_aligned16(conv_w),
                 HDCM_EALIGN);
  HDCM_CHECK_ARG(ws != nullptr && ws_bytes >= hdcm_norm_conv_bwd_workspace_bytes(B, L, D), HDCM_EWORKSPACE);
  HDCM_CHECK_ARG(((uintptr_t)ws & 255u) == 0, HDCM_EALIGN);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HDCM_F32)
    return launch_bwd<float>(grad_out, g_batch_stride, g_row_stride, x, x_batch_stride, x_row_stride, ln_w, ln_b,
                             conv_w, dx, dx_batch_stride, dx_row_stride, d_ln_w, d_ln_b, d_conv_w, d_conv_b, ws, B,
                             L, D, eps, s);
  return launch_bwd<bf16_t>(grad_out, g_batch_stride, g_row_stride, x, x_batch_stride, x_row_stride, ln_w, ln_b,
                            conv_w, dx, dx_batch_stride, dx_row_stride, d_ln_w, d_ln_b, d_conv_w, d_conv_b, ws, B, L,
                            D, eps, s);
}
