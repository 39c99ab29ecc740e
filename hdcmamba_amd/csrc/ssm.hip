// Diagonal selective scan over d_state channels for gfx950.
//
// Semantics (hdcmamba/model.py:175-233, intended form): per channel d and row t,
//   dt = softplus(dt_raw) with threshold 20 (log(1+exp(x)) below it),
//   a_t = exp(dt * A_d), A_d = -exp(A_log_d),  u_t = dt * b * x,
//   h_t = a_t * h_{t-1} + u_t,  y_t = h_t.
// All state is fp32; y is rounded once to the activation dtype.
//
// The recurrence is the associative scan of pairs (a, u) under
//   (a1, u1) then (a2, u2)  =  (a1*a2, a2*u1 + u2),
// so a wave scans 64 consecutive rows of one channel with lanes = rows in six
// shuffle steps instead of a 64-step serial loop.  Rows are cut into tiles of 64:
//   1. ssm_tile_kernel<SUMMARY>: stage a tile's dt/x/b for 64 channels through LDS as
//      (a, u) pairs, scan each channel, keep the tile total (A, H) [b][channel][tile].
//   2. ssm_carry_kernel: per channel, scan the tile totals (lanes = groups of tiles) to
//      get the state entering every tile, h_in[b][channel][tile], and h_final.
//   3. ssm_tile_kernel<OUTPUT>: rescan each tile, y_t = U_t + A_t * h_in, staged back
//      through LDS for 128-bit row stores.
#include "hdcm_common.h"

using namespace hdcm;

namespace {

constexpr int kTile = 64;      // rows per tile (= lanes of a wave)
constexpr int kCh = 64;        // channels per workgroup
constexpr int kThreads = 256;  // 4 waves, 16 channels each
constexpr int kPitch = kCh + 1;

// BWD: the adjoint recurrence g_t = a_{t+1} g_{t+1} + gy_t of the backward, scanned over
// the rows in reverse (tile k holds rows L-1-64k downwards): the pair of reversed row
// tau = L-1-t is (a_{t+1}, gy_t), the decay taken from the dt of the row after t.  y then
// receives g.
template <typename T, bool OUTPUT, bool BWD>
__global__ __launch_bounds__(kThreads) void ssm_tile_kernel(
    const T* __restrict__ projs, int64_t prs, const T* __restrict__ A_log,
    float* __restrict__ tot_a, float* __restrict__ tot_h, const float* __restrict__ hin,
    T* __restrict__ y, int64_t yrs, float* __restrict__ h_final, int L, int ds, int ntiles,
    const T* __restrict__ gy, int64_t gyrs) {
  constexpr int E = Vec<T>::N;
  constexpr int GPR = kCh / E;                       // 16-byte groups per row per block
  constexpr int ITEMS = kTile * GPR / kThreads;      // (row, group) items per thread
  __shared__ float sa[kTile * kPitch];
  __shared__ float su[kTile * kPitch];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int tile = blockIdx.x, c0 = blockIdx.y * kCh, b = blockIdx.z;
  const int t0 = tile * kTile;
  const int tlen = min(kTile, L - t0);
  const int nch = min(kCh, ds - c0);
  const T* base = projs + ((int64_t)b * L + t0) * prs + c0;
  // forward row of tile row i
  auto trow = [&](int i) { return BWD ? L - 1 - (t0 + i) : t0 + i; };

  // Stage (a, u) pairs.  Rows past the tile or channels past ds get the identity (1, 0).
  uint4 rd[ITEMS], rx[ITEMS], rb[ITEMS];  // BWD: dt of the next row, unused, gy
  // every item of this thread covers the same column group (kThreads is a multiple of GPR)
  const int cg0 = tid % GPR;
  float negA[E];
  {
    float al[E] = {};
    if (cg0 * E < nch) load16<T>(A_log + c0 + cg0 * E, al);
#pragma unroll
    for (int e = 0; e < E; ++e) negA[e] = -fexp(al[e]);
  }
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    const int idx = tid + kThreads * k;
    const int i = idx / GPR, cg = idx % GPR;
    const bool ok = i < tlen && cg * E < nch;
    if constexpr (BWD) {
      const int t = trow(i);
      const bool nxt = ok && t + 1 < L;
      rd[k] = nxt ? ldg16(projs + ((int64_t)b * L + t + 1) * prs + c0 + cg * E) : make_uint4(0, 0, 0, 0);
      rb[k] = ok ? ldg16(gy + ((int64_t)b * L + t) * gyrs + c0 + cg * E) : make_uint4(0, 0, 0, 0);
    } else {
      const T* r = base + (int64_t)i * prs + cg * E;
      rd[k] = ok ? ldg16(r) : make_uint4(0, 0, 0, 0);
      rx[k] = ok ? ldg16(r + ds) : make_uint4(0, 0, 0, 0);
      rb[k] = ok ? ldg16(r + 2 * ds) : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    const int idx = tid + kThreads * k;
    const int i = idx / GPR, cg = idx % GPR;
    const bool ok = i < tlen && cg * E < nch;
    float d[E], xv[E], bv[E];
    unpack16<T>(rd[k], d);
    unpack16<T>(rb[k], bv);
    if constexpr (BWD) {
      const bool nxt = ok && trow(i) + 1 < L;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        sa[i * kPitch + cg * E + e] = nxt ? fexp(softplus20(d[e]) * negA[e]) : 1.0f;
        su[i * kPitch + cg * E + e] = ok ? bv[e] : 0.0f;
      }
    } else {
      unpack16<T>(rx[k], xv);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float dt = softplus20(d[e]);
        sa[i * kPitch + cg * E + e] = ok ? fexp(dt * negA[e]) : 1.0f;
        su[i * kPitch + cg * E + e] = ok ? dt * bv[e] * xv[e] : 0.0f;
      }
    }
  }
  __syncthreads();

  // Wave w scans channels w + 4*(k*kNC + c) for c < kNC, kNC at a time; lane = row.
  // Channels past nch scan the identity pairs staged above and are never written.
  constexpr int kNC = 4;
  constexpr int kWaves = kThreads / kWave;
  const int64_t tb = (int64_t)b * ds;
  for (int cb = w; cb < nch; cb += kWaves * kNC) {
    float a[kNC], u[kNC];
#pragma unroll
    for (int c = 0; c < kNC; ++c) {
      const int ch = cb + kWaves * c;
      a[c] = ch < kCh ? sa[lane * kPitch + ch] : 1.0f;
      u[c] = ch < kCh ? su[lane * kPitch + ch] : 0.0f;
    }
    scan_pairs<kNC>(a, u);
#pragma unroll
    for (int c = 0; c < kNC; ++c) {
      const int ch = cb + kWaves * c;
      if (ch >= nch) continue;
      const int64_t ci = (tb + c0 + ch) * ntiles + tile;  // [b][channel][tile]
      if constexpr (!OUTPUT) {
        if (lane == kWave - 1) {
          tot_a[ci] = a[c];
          tot_h[ci] = u[c];
        }
      } else {
        const float h = u[c] + a[c] * hin[ci];
        su[lane * kPitch + ch] = h;
        if (h_final != nullptr && tile == ntiles - 1 && lane == tlen - 1) h_final[tb + c0 + ch] = h;
      }
    }
  }
  if constexpr (OUTPUT) {
    __syncthreads();
    T* ybase = y + (int64_t)b * L * yrs + c0;
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const int idx = tid + kThreads * k;
      const int i = idx / GPR, cg = idx % GPR;
      if (i < tlen && cg * E < nch) {
        float v[E];
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = su[i * kPitch + cg * E + e];
        store16<T>(ybase + (int64_t)trow(i) * yrs + cg * E, v);
      }
    }
  }
}

// One wave per (channel, batch): lanes own consecutive groups of tiles.
__global__ __launch_bounds__(kWave) void ssm_carry_kernel(const float* __restrict__ tot_a,
                                                          const float* __restrict__ tot_h,
                                                          const float* __restrict__ h0,
                                                          float* __restrict__ hin,
                                                          float* __restrict__ h_final, int ds,
                                                          int ntiles) {
  const int c = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int64_t row = ((int64_t)b * ds + c) * ntiles;
  const int per = (ntiles + kWave - 1) / kWave;
  const int n0 = min(lane * per, ntiles), n1 = min(n0 + per, ntiles);
  float A = 1.0f, Hs = 0.0f;
  for (int n = n0; n < n1; ++n) {
    const float a = tot_a[row + n];
    Hs = a * Hs + tot_h[row + n];
    A = A * a;
  }
  // exclusive scan of the lane aggregates
  float ia = A, ih = Hs;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const float ap = __shfl_up(ia, off, kWave);
    const float hp = __shfl_up(ih, off, kWave);
    if (lane >= off) {
      ih = ia * hp + ih;
      ia = ia * ap;
    }
  }
  float ea = __shfl_up(ia, 1, kWave), eh = __shfl_up(ih, 1, kWave);
  if (lane == 0) {
    ea = 1.0f;
    eh = 0.0f;
  }
  const float init = h0 ? h0[(int64_t)b * ds + c] : 0.0f;
  float h = ea * init + eh;
  for (int n = n0; n < n1; ++n) {
    hin[row + n] = h;
    h = tot_a[row + n] * h + tot_h[row + n];
  }
  if (h_final != nullptr && n1 == ntiles && n0 < n1) h_final[(int64_t)b * ds + c] = h;
}

inline int64_t ssm_tiles(int64_t L) { return (L + kTile - 1) / kTile; }

template <typename T>
int launch(const void* projs, int64_t prs, const void* A_log, const float* h0, void* y,
           int64_t yrs, float* h_final, void* ws, int64_t B, int64_t L, int64_t ds,
           hipStream_t s) {
  const int64_t nt = ssm_tiles(L);
  const int64_t n = B * nt * ds;
  float* ta = (float*)ws;
  float* th = ta + n;
  float* hin = th + n;
  const dim3 grid((unsigned)nt, (unsigned)((ds + kCh - 1) / kCh), (unsigned)B);
  HDCM_LAUNCH((ssm_tile_kernel<T, false, false>), grid, dim3(kThreads), 0, s, (const T*)projs, prs,
                     (const T*)A_log, ta, th, (const float*)nullptr, (T*)nullptr, (int64_t)0,
                     (float*)nullptr, (int)L, (int)ds, (int)nt, (const T*)nullptr, (int64_t)0);
  int st = hdcm_launch_status();
  if (st) return st;
  HDCM_LAUNCH(ssm_carry_kernel, dim3((unsigned)ds, (unsigned)B), dim3(kWave), 0, s, ta, th, h0,
                     hin, h_final, (int)ds, (int)nt);
  st = hdcm_launch_status();
  if (st) return st;
  HDCM_LAUNCH((ssm_tile_kernel<T, true, false>), grid, dim3(kThreads), 0, s, (const T*)projs, prs,
                     (const T*)A_log, (float*)nullptr, (float*)nullptr, hin, (T*)y, yrs,
                     (float*)nullptr, (int)L, (int)ds, (int)nt, (const T*)nullptr, (int64_t)0);
  return hdcm_launch_status();
}

}  // namespace

extern "C" size_t hdcm_ssm_workspace_bytes(int64_t B, int64_t L, int64_t ds) {
  if (B <= 0 || L <= 0 || ds <= 0) return 0;
  return (size_t)(3 * B * ssm_tiles(L) * ds) * sizeof(float);
}

// Argument checks of the forward entry points, everything but the workspace (also used by
// other sources of the library that run these kernels).
int hdcm_ssm_check_fwd(const void* projs, int64_t proj_row_stride, const void* A_log, const void* y,
                       int64_t y_row_stride, int64_t B, int64_t L, int64_t ds, int dtype) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(A_log && ((projs && y) || B == 0 || L == 0), HDCM_EINVAL);  // empty: NULL data allowed
  HDCM_CHECK_ARG(B >= 0 && L >= 0 && ds > 0, HDCM_EINVAL);
  HDCM_CHECK_ARG(proj_row_stride >= 3 * ds && y_row_stride >= ds, HDCM_EINVAL);
  const int E = 16 / hdcm_elt_size(dtype);
  HDCM_CHECK_ARG(ds % E == 0 && proj_row_stride % E == 0 && y_row_stride % E == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(hdcm_aligned16(projs) && hdcm_aligned16(y) && hdcm_aligned16(A_log), HDCM_EALIGN);
  HDCM_CHECK_ARG(B <= 65535 && ssm_tiles(L) < ((int64_t)1 << 31) && ds <= 65535, HDCM_EUNSUPPORTED);
  return HDCM_OK;
}

// The forward's launches on a checked, non-empty input with a workspace of
// hdcm_ssm_workspace_bytes(B, L, ds) bytes at `ws` (4-byte aligned).
int hdcm_ssm_launch_fwd(const void* projs, int64_t proj_row_stride, const void* A_log, const float* h0, void* y,
                        int64_t y_row_stride, float* h_final, void* ws, int64_t B, int64_t L, int64_t ds, int dtype,
                        hipStream_t s) {
  if (dtype == HDCM_F32)
    return launch<float>(projs, proj_row_stride, A_log, h0, y, y_row_stride, h_final, ws, B, L, ds, s);
  return launch<bf16_t>(projs, proj_row_stride, A_log, h0, y, y_row_stride, h_final, ws, B, L, ds, s);
}

extern "C" int hdcm_ssm_fwd(const void* projs, int64_t proj_row_stride, const void* A_log,
                            const float* h0, void* y, int64_t y_row_stride, float* h_final,
                            void* ws, size_t ws_bytes, int64_t B, int64_t L, int64_t ds, int dtype,
                            void* stream) {
  const int st = hdcm_ssm_check_fwd(projs, proj_row_stride, A_log, y, y_row_stride, B, L, ds, dtype);
  if (st) return st;
  if (B == 0 || L == 0) return HDCM_OK;
  HDCM_CHECK_ARG(ws != nullptr && ws_bytes >= hdcm_ssm_workspace_bytes(B, L, ds), HDCM_EWORKSPACE);
  HDCM_CHECK_ARG(((uintptr_t)ws & 3u) == 0, HDCM_EALIGN);
  return hdcm_ssm_launch_fwd(projs, proj_row_stride, A_log, h0, y, y_row_stride, h_final, ws, B, L, ds, dtype,
                             (hipStream_t)stream);
}

// ------------------------------------------------------------------------- backward
// Gradient of the scan above, given gy = dLoss/dy and h = y (the forward's output, h_{-1} = 0):
//   g_t     = gy_t + a_{t+1} g_{t+1}                      (adjoint scan, ssm_tile_kernel<BWD>)
//   d dt_t  = g_t (h_{t-1} a_t A + b_t x_t),  d dt_raw = d dt * (dt_raw > 20 ? 1 : sigmoid(dt_raw))
//   d b_t   = g_t dt_t x_t,  d x_t = g_t dt_t b_t
//   d A_log = sum_t g_t h_{t-1} a_t dt_t A               (A = -exp(A_log))
// ssm_grad_kernel computes the row terms (a fixed grid of workgroups striding over rows, one
// thread per 16-byte column group) and each workgroup's sums for d A_log, which
// colsum_kernel adds in a fixed order.
namespace {

constexpr int kGradMaxBlocks = 1024;

int64_t grad_blocks(int64_t rows, int64_t ds, int E) {
  const int64_t gpr = ds / E;
  const int64_t rows_per = kThreads / gpr;
  const int64_t need = (rows + rows_per - 1) / rows_per;
  return need < kGradMaxBlocks ? (need > 0 ? need : 1) : kGradMaxBlocks;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void ssm_grad_kernel(
    const T* __restrict__ projs, int64_t prs, const T* __restrict__ A_log, const T* __restrict__ h, int64_t hrs,
    const T* __restrict__ g, int64_t grs, T* __restrict__ dprojs, int64_t dprs, float* __restrict__ part, int64_t rows,
    int L, int ds) {
  constexpr int E = Vec<T>::N;
  extern __shared__ float sred[];  // [kThreads / GPR][ds]
  const int GPR = ds / E, rows_per = kThreads / GPR;
  const int tid = threadIdx.x, cg = tid % GPR, rr = tid / GPR;
  const bool act = rr < rows_per;
  float A[E], accA[E];
  {
    float al[E];
    load16<T>(A_log + cg * E, al);
#pragma unroll
    for (int e = 0; e < E; ++e) A[e] = -fexp(al[e]), accA[e] = 0.f;
  }
  const int64_t stride = (int64_t)gridDim.x * rows_per;
  for (int64_t row = (int64_t)blockIdx.x * rows_per + rr; act && row < rows; row += stride) {
    const int t = (int)(row % L);
    const T* pr = projs + row * prs + cg * E;
    const uint4 rraw = ldg16(pr), rx = ldg16(pr + ds), rb = ldg16(pr + 2 * ds);
    const uint4 rg = ldg16(g + row * grs + cg * E);
    const uint4 rh = t > 0 ? ldg16(h + (row - 1) * hrs + cg * E) : make_uint4(0, 0, 0, 0);
    float raw[E], xv[E], bv[E], gv[E], hp[E], dr[E], dx[E], db[E];
    unpack16<T>(rraw, raw);
    unpack16<T>(rx, xv);
    unpack16<T>(rb, bv);
    unpack16<T>(rg, gv);
    unpack16<T>(rh, hp);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float dt = softplus20(raw[e]);
      const float a = fexp(dt * A[e]);
      const float ddt = gv[e] * (hp[e] * a * A[e] + bv[e] * xv[e]);
      dr[e] = ddt * (raw[e] > 20.f ? 1.f : frcp(1.f + fexp(-raw[e])));
      dx[e] = gv[e] * dt * bv[e];
      db[e] = gv[e] * dt * xv[e];
      accA[e] += gv[e] * hp[e] * a * dt * A[e];
    }
    T* dp = dprojs + row * dprs + cg * E;
    store16<T>(dp, dr);
    store16<T>(dp + ds, dx);
    store16<T>(dp + 2 * ds, db);
  }
  // this workgroup's d A_log: rows of threads in turn through LDS (fixed order)
  if (act) {
#pragma unroll
    for (int e = 0; e < E; ++e) sred[rr * ds + cg * E + e] = accA[e];
  }
  __syncthreads();
  for (int c = tid; c < ds; c += kThreads) {
    float sum = 0.f;
    for (int k = 0; k < rows_per; ++k) sum += sred[k * ds + c];
    part[(int64_t)blockIdx.x * ds + c] = sum;
  }
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

template <typename T>
int launch_bwd(const void* projs, int64_t prs, const void* A_log, const void* h, int64_t hrs, const void* gy,
               int64_t gyrs, void* dprojs, int64_t dprs, float* dA_log, void* ws, int64_t B, int64_t L, int64_t ds,
               hipStream_t s) {
  constexpr int E = Vec<T>::N;
  const int64_t nt = ssm_tiles(L);
  const int64_t n = B * nt * ds;
  float* ta = (float*)ws;
  float* th = ta + n;
  float* hin = th + n;
  T* g = (T*)((char*)ws + align256((size_t)3 * n * sizeof(float)));
  float* part = (float*)((char*)g + align256((size_t)B * L * ds * sizeof(T)));
  const dim3 grid((unsigned)nt, (unsigned)((ds + kCh - 1) / kCh), (unsigned)B);
  HDCM_LAUNCH((ssm_tile_kernel<T, false, true>), grid, dim3(kThreads), 0, s, (const T*)projs, prs,
                     (const T*)A_log, ta, th, (const float*)nullptr, (T*)nullptr, (int64_t)0, (float*)nullptr,
                     (int)L, (int)ds, (int)nt, (const T*)gy, gyrs);
  int st = hdcm_launch_status();
  if (st) return st;
  HDCM_LAUNCH(ssm_carry_kernel, dim3((unsigned)ds, (unsigned)B), dim3(kWave), 0, s, ta, th,
                     (const float*)nullptr, hin, (float*)nullptr, (int)ds, (int)nt);
  st = hdcm_launch_status();
  if (st) return st;
  HDCM_LAUNCH((ssm_tile_kernel<T, true, true>), grid, dim3(kThreads), 0, s, (const T*)projs, prs,
                     (const T*)A_log, (float*)nullptr, (float*)nullptr, hin, g, ds, (float*)nullptr, (int)L,
                     (int)ds, (int)nt, (const T*)gy, gyrs);
  st = hdcm_launch_status();
  if (st) return st;
  const int64_t nb = grad_blocks(B * L, ds, E);
  const int rows_per = (int)(kThreads / (ds / E));
  HDCM_LAUNCH((ssm_grad_kernel<T>), dim3((unsigned)nb), dim3(kThreads),
                     (size_t)rows_per * ds * sizeof(float), s, (const T*)projs, prs, (const T*)A_log, (const T*)h,
                     hrs, (const T*)g, ds, (T*)dprojs, dprs, part, B * L, (int)L, (int)ds);
  st = hdcm_launch_status();
  if (st) return st;
  return hdcm_colsum(part, ds, (int)nb, (int)ds, (int)ds, 0, dA_log, (int)ds, nullptr, s);
}

}  // namespace

extern "C" size_t hdcm_ssm_bwd_workspace_bytes(int64_t B, int64_t L, int64_t ds, int dtype) {
  if (B <= 0 || L <= 0 || ds <= 0 || (dtype != HDCM_F32 && dtype != HDCM_BF16)) return 0;
  const int esz = hdcm_elt_size(dtype);
  return align256((size_t)3 * B * ssm_tiles(L) * ds * sizeof(float)) + align256((size_t)B * L * ds * esz) +
         (size_t)grad_blocks(B * L, ds, 16 / esz) * ds * sizeof(float);
}

extern "C" int hdcm_ssm_bwd(const void* projs, int64_t proj_row_stride, const void* A_log, const void* h,
                            int64_t h_row_stride, const void* gy, int64_t gy_row_stride, void* dprojs,
                            int64_t dprojs_row_stride, float* dA_log, void* ws, size_t ws_bytes, int64_t B, int64_t L,
                            int64_t ds, int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(A_log && dA_log && ((projs && h && gy && dprojs) || B == 0 || L == 0), HDCM_EINVAL);
  HDCM_CHECK_ARG(B >= 0 && L >= 0 && ds > 0, HDCM_EINVAL);
  const int E = 16 / hdcm_elt_size(dtype);
  HDCM_CHECK_ARG(ds % E == 0 && hdcm_aligned16(A_log), HDCM_EALIGN);
  HDCM_CHECK_ARG(B <= 65535 && ssm_tiles(L) < ((int64_t)1 << 31) && ds <= 65535 && ds / E <= kThreads,
                 HDCM_EUNSUPPORTED);
  hipStream_t s = (hipStream_t)stream;
  if (B == 0 || L == 0)  // no rows: d A_log is zero
    return hdcm_colsum(nullptr, ds, 0, (int)ds, (int)ds, 0, dA_log, (int)ds, nullptr, s);
  HDCM_CHECK_ARG(proj_row_stride >= 3 * ds && h_row_stride >= ds && gy_row_stride >= ds &&
                     dprojs_row_stride >= 3 * ds,
                 HDCM_EINVAL);
  HDCM_CHECK_ARG(proj_row_stride % E == 0 && h_row_stride % E == 0 && gy_row_stride % E == 0 &&
                     dprojs_row_stride % E == 0,
                 HDCM_EALIGN);
  HDCM_CHECK_ARG(hdcm_aligned16(projs) && hdcm_aligned16(h) && hdcm_aligned16(gy) && hdcm_aligned16(dprojs),
                 HDCM_EALIGN);
  HDCM_CHECK_ARG(ws != nullptr && ws_bytes >= hdcm_ssm_bwd_workspace_bytes(B, L, ds, dtype), HDCM_EWORKSPACE);
  HDCM_CHECK_ARG(((uintptr_t)ws & 255u) == 0, HDCM_EALIGN);
  if (dtype == HDCM_F32)
    return launch_bwd<float>(projs, proj_row_stride, A_log, h, h_row_stride, gy, gy_row_stride, dprojs,
                             dprojs_row_stride, dA_log, ws, B, L, ds, s);
  return launch_bwd<bf16_t>(projs, proj_row_stride, A_log, h, h_row_stride, gy, gy_row_stride, dprojs,
                            dprojs_row_stride, dA_log, ws, B, L, ds, s);
}
