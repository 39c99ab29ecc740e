// Backward of the slot memory's GroupNorm + gate and of its feature map, for gfx950.
//
// Forward (hdcmamba/model.py:261-262, 274-295, intended form), per token and head h over
// the head's hd values:  out = (x^ * w + b) * s,  x^ = (y - mean) * rstd,  s = sigmoid(gate),
// with y the slot recurrence's output over phi(q), phi(k), v.  Given dout:
//   d gate = dout * (x^ w + b) * s (1 - s)
//   d x^   = dout * s * w,   dy = rstd * (d x^ - mean(d x^) - x^ mean(d x^ * x^))
//   d w    = sum over tokens of dout * s * x^,   d b = sum over tokens of dout * s
// The recurrence's own gradient is the recurrence again (hdcm_slot_attend_fwd on the
// operands this file stages): with Z = [dy | v | phi(k) | phi(q)] per row,
//   d phi(q) = attend(q=dy, k=v, v=phi(k)),  d v = attend(q=phi(k), k=phi(q), v=dy) backwards,
//   d phi(k) = attend(q=v, k=dy, v=phi(q)) backwards,
// and d q = d phi(q) * phi'(q), d k = d phi(k) * phi'(k), phi'(z) = 1 (z > 0) else exp(z).
//
// gnorm_gate_bwd_kernel: one wave per (token, head) at a time, lane i holding column i (and
// i + 64 when hd > 64); the waves of the grid stride over (token, head) pairs with a stride
// that is a multiple of H, so a wave always meets the same head and keeps that head's d w,
// d b column sums in registers; colsum_kernel adds the waves' sums in a fixed order.  Used
// for head widths whose 16-byte groups do not form a power-of-two lane group (hd = 96);
// gnorm_gate_bwd_rows_kernel below covers the others.  The feature-map kernels are
// elementwise over 16-byte groups.
#include "hdcm_common.h"

using namespace hdcm;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kWavesPerHead = 256;  // waves of the grid that share one head

template <typename T>
__device__ __forceinline__ float ld1(const T* p) {
  return to_f<T>(*p);
}

template <typename T, int HD>
__global__ __launch_bounds__(kThreads) void gnorm_gate_bwd_kernel(
    const T* __restrict__ y, int64_t y_rs, const T* __restrict__ gate, int64_t g_rs, const T* __restrict__ gn_w,
    const T* __restrict__ gn_b, float eps, const T* __restrict__ dout, int64_t do_rs, T* __restrict__ dy,
    int64_t dy_rs, T* __restrict__ dgate, int64_t dg_rs, float* __restrict__ part, int64_t rows, int H) {
  constexpr int NV = (HD + kWave - 1) / kWave;  // columns per lane
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = (int64_t)blockIdx.x * kWaves + threadIdx.x / kWave;
  const int64_t nwaves = (int64_t)gridDim.x * kWaves;  // a multiple of H
  const int h = (int)(wave % H);
  float w[NV], bb[NV], aw[NV], ab[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c = lane + kWave * k;
    const bool ok = c < HD;
    w[k] = ok ? ld1(gn_w + h * HD + c) : 0.f;
    bb[k] = ok ? ld1(gn_b + h * HD + c) : 0.f;
    aw[k] = ab[k] = 0.f;
  }
  for (int64_t pr = wave; pr < rows * H; pr += nwaves) {
    const int64_t row = pr / H;
    const int64_t col0 = (int64_t)h * HD;
    float yv[NV], gv[NV], dv[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = lane + kWave * k;
      const bool ok = c < HD;
      yv[k] = ok ? ld1(y + row * y_rs + col0 + c) : 0.f;
      gv[k] = ok ? ld1(gate + row * g_rs + col0 + c) : 0.f;
      dv[k] = ok ? ld1(dout + row * do_rs + col0 + c) : 0.f;
    }
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) s += yv[k];
    const float mean = wave_total(s) * (1.0f / HD);
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const bool ok = lane + kWave * k < HD;
      yv[k] = ok ? yv[k] - mean : 0.f;
      q += yv[k] * yv[k];
    }
    const float rstd = rsqrtf(wave_total(q) * (1.0f / HD) + eps);
    float dxh[NV], xh[NV], sa = 0.f, sb = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const bool ok = lane + kWave * k < HD;
      xh[k] = yv[k] * rstd;
      const float sg = frcp(1.0f + fexp(-gv[k]));
      const float yn = xh[k] * w[k] + bb[k];
      const float dyn = dv[k] * sg;
      gv[k] = dv[k] * yn * sg * (1.0f - sg);  // d gate
      aw[k] += ok ? dyn * xh[k] : 0.f;
      ab[k] += ok ? dyn : 0.f;
      dxh[k] = ok ? dyn * w[k] : 0.f;
      sa += dxh[k];
      sb += dxh[k] * xh[k];
    }
    const float ma = wave_total(sa) * (1.0f / HD), mb = wave_total(sb) * (1.0f / HD);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = lane + kWave * k;
      if (c < HD) {
        dy[row * dy_rs + col0 + c] = from_f<T>(rstd * (dxh[k] - ma - xh[k] * mb));
        dgate[row * dg_rs + col0 + c] = from_f<T>(gv[k]);
      }
    }
  }
  // this wave's column sums: part[wave][2][HD]
  float* pw = part + wave * 2 * HD;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c = lane + kWave * k;
    if (c < HD) {
      pw[c] = aw[k];
      pw[HD + c] = ab[k];
    }
  }
}

// Row-stripe form of the same backward, for heads of GL = HD / E lanes with GL a power of
// two (E values of a 16-byte group per lane).  A workgroup's four waves share one stripe of
// 64 groups of the row (stripe = blockIdx % nstripe) and stride over tokens, so each lane
// keeps its E columns' d w, d b sums in registers; the head statistics are GL-lane group
// sums.  Loads and stores are 16 bytes per lane.  The four waves' sums are added in LDS in
// wave order and each workgroup leaves part[m][2][dm] (m = blockIdx / nstripe) for
// colsum_kernel.  The next token's three groups are loaded before the current one is used.
template <typename T, int HD>
__global__ __launch_bounds__(kThreads) void gnorm_gate_bwd_rows_kernel(
    const T* __restrict__ y, int64_t y_rs, const T* __restrict__ gate, int64_t g_rs, const T* __restrict__ gn_w,
    const T* __restrict__ gn_b, float eps, const T* __restrict__ dout, int64_t do_rs, T* __restrict__ dy,
    int64_t dy_rs, T* __restrict__ dgate, int64_t dg_rs, float* __restrict__ part, int64_t rows, int dm,
    int nstripe) {
  constexpr int E = Vec<T>::N;
  constexpr int GL = HD / E;
  constexpr float kInvHD = 1.0f / HD;
  __shared__ float red[kWaves][2][kWave * E];
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int stripe = (int)(blockIdx.x % (unsigned)nstripe);
  const int64_t m = blockIdx.x / (unsigned)nstripe;
  const int64_t nblk = gridDim.x / (unsigned)nstripe;
  const int G = dm / E;
  const int cg = stripe * kWave + lane;
  const bool ok = cg < G;
  const int64_t c0 = (int64_t)cg * E;
  float w[E], bb[E], aw[E], ab[E];
#pragma unroll
  for (int e = 0; e < E; ++e) aw[e] = ab[e] = w[e] = bb[e] = 0.f;
  if (ok) {
    load16<T>(gn_w + c0, w);
    load16<T>(gn_b + c0, bb);
  }
  const uint4 zero = make_uint4(0, 0, 0, 0);
  const int64_t tstep = nblk * kWaves;
  int64_t t = m * kWaves + wv;
  uint4 ry = zero, rg = zero, rd = zero;
  if (ok && t < rows) {
    ry = ldg16(y + t * y_rs + c0);
    rg = ldg16(gate + t * g_rs + c0);
    rd = ldg16(dout + t * do_rs + c0);
  }
  for (; t < rows; t += tstep) {
    float yv[E], gv[E], dv[E];
    unpack16<T>(ry, yv);
    unpack16<T>(rg, gv);
    unpack16<T>(rd, dv);
    const int64_t tn = t + tstep;
    if (ok && tn < rows) {
      ry = ldg16(y + tn * y_rs + c0);
      rg = ldg16(gate + tn * g_rs + c0);
      rd = ldg16(dout + tn * do_rs + c0);
    }
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) s += yv[e];
    const float mean = group_sum<GL>(s) * kInvHD;
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      yv[e] -= mean;
      q += yv[e] * yv[e];
    }
    const float rstd = rsqrtf(group_sum<GL>(q) * kInvHD + eps);
    float dxh[E], sa = 0.f, sb = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float xh = yv[e] * rstd;
      const float sg = frcp(1.0f + fexp(-gv[e]));
      const float yn = xh * w[e] + bb[e];
      const float dyn = dv[e] * sg;
      gv[e] = dv[e] * yn * sg * (1.0f - sg);  // d gate
      aw[e] += dyn * xh;
      ab[e] += dyn;
      dxh[e] = dyn * w[e];
      sa += dxh[e];
      sb += dxh[e] * xh;
      yv[e] = xh;
    }
    const float ma = group_sum<GL>(sa) * kInvHD, mb = group_sum<GL>(sb) * kInvHD;
    if (ok) {
#pragma unroll
      for (int e = 0; e < E; ++e) dxh[e] = rstd * (dxh[e] - ma - yv[e] * mb);
      store16<T>(dy + t * dy_rs + c0, dxh);
      store16<T>(dgate + t * dg_rs + c0, gv);
    }
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    red[wv][0][lane * E + e] = aw[e];
    red[wv][1][lane * E + e] = ab[e];
  }
  __syncthreads();
  float* pm = part + m * 2 * (int64_t)dm + (int64_t)stripe * kWave * E;
  const int width = min(kWave, G - stripe * kWave) * E;  // valid columns of this stripe
  for (int i = threadIdx.x; i < 2 * kWave * E; i += kThreads) {
    const int j = i / (kWave * E), c = i % (kWave * E);
    if (c < width) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < kWaves; ++k) acc += red[k][j][c];
      pm[(int64_t)j * dm + c] = acc;
    }
  }
}

// Z[row] = [-- | v | round(phi(k)) | round(phi(q))] (the first block, dy, is written by the
// GroupNorm backward).  One thread per 16-byte group of a dm-wide block, grid-stride.
template <typename T>
__global__ __launch_bounds__(kThreads) void phi_prep_kernel(const T* __restrict__ projs, int64_t prs, int q_col,
                                                            T* __restrict__ z, int64_t zrs, int64_t rows, int dm) {
  constexpr int E = Vec<T>::N;
  const int G = dm / E;
  const int64_t n = rows * G;
  for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < n; idx += (int64_t)gridDim.x * kThreads) {
    const int64_t row = idx / G;
    const int cg = (int)(idx % G);
    const T* pr = projs + row * prs + q_col + cg * E;
    T* zr = z + row * zrs + cg * E;
    const uint4 rq = ldg16(pr), rk = ldg16(pr + dm), rv = ldg16(pr + 2 * dm);
    float f[E];
    *reinterpret_cast<uint4*>(zr + dm) = rv;
    unpack16<T>(rk, f);
#pragma unroll
    for (int e = 0; e < E; ++e) f[e] = phi_f(f[e]);
    store16<T>(zr + 2 * dm, f);
    unpack16<T>(rq, f);
#pragma unroll
    for (int e = 0; e < E; ++e) f[e] = phi_f(f[e]);
    store16<T>(zr + 3 * dm, f);
  }
}

// In place on the q and k column blocks of dprojs: d q = d phi(q) * phi'(q), d k likewise.
template <typename T>
__global__ __launch_bounds__(kThreads) void phi_chain_kernel(const T* __restrict__ projs, int64_t prs, int q_col,
                                                             T* __restrict__ dprojs, int64_t drs, int64_t rows,
                                                             int dm) {
  constexpr int E = Vec<T>::N;
  const int G = 2 * dm / E;  // q and k blocks are adjacent
  const int64_t n = rows * G;
  for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < n; idx += (int64_t)gridDim.x * kThreads) {
    const int64_t row = idx / G;
    const int cg = (int)(idx % G);
    float z[E], d[E];
    unpack16<T>(ldg16(projs + row * prs + q_col + cg * E), z);
    T* dp = dprojs + row * drs + q_col + cg * E;
    unpack16<T>(ldg16(dp), d);
#pragma unroll
    for (int e = 0; e < E; ++e) d[e] *= z[e] > 0.f ? 1.0f : fexp(z[e]);
    store16<T>(dp, d);
  }
}

unsigned grid_for(int64_t n) {
  const int64_t b = (n + kThreads - 1) / kThreads;
  return (unsigned)(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

constexpr int kStripeBlocks = 512;  // workgroups per row stripe, row-stripe kernel

// Row-stripe kernel for this head width and element size?
bool stripe_form(int64_t hd, int esz) {
  const int64_t gl = hd * esz / 16;
  return hd * esz % 16 == 0 && gl >= 1 && gl <= kWave && (gl & (gl - 1)) == 0;
}

}  // namespace

extern "C" size_t hdcm_gnorm_gate_bwd_workspace_bytes(int64_t dm, int64_t H) {
  if (dm <= 0 || H <= 0 || dm % H) return 0;
  const size_t per_head = (size_t)H * kWavesPerHead * 2 * (size_t)(dm / H) * sizeof(float);
  const size_t stripes = (size_t)kStripeBlocks * 2 * (size_t)dm * sizeof(float);
  return per_head > stripes ? per_head : stripes;
}

extern "C" int hdcm_gnorm_gate_bwd(const void* y, int64_t y_row_stride, const void* gate, int64_t gate_row_stride,
                                   const void* gn_w, const void* gn_b, float eps, const void* dout,
                                   int64_t dout_row_stride, void* dy, int64_t dy_row_stride, void* dgate,
                                   int64_t dgate_row_stride, float* dgn_w, float* dgn_b, void* ws, size_t ws_bytes,
                                   int64_t rows, int64_t dm, int64_t H, int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(gn_w && gn_b && dgn_w && dgn_b && ((y && gate && dout && dy && dgate) || rows == 0), HDCM_EINVAL);
  HDCM_CHECK_ARG(rows >= 0 && dm > 0 && H > 0 && dm % H == 0, HDCM_EINVAL);
  const int64_t hd = dm / H;
  HDCM_CHECK_ARG(hd >= 16 && hd <= 128 && hd % 16 == 0, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(H <= 65535, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(ws != nullptr && ws_bytes >= hdcm_gnorm_gate_bwd_workspace_bytes(dm, H), HDCM_EWORKSPACE);
  HDCM_CHECK_ARG(((uintptr_t)ws & 15u) == 0, HDCM_EALIGN);
  hipStream_t s = (hipStream_t)stream;
  if (stripe_form(hd, hdcm_elt_size(dtype))) {
    const int E = 16 / hdcm_elt_size(dtype);
    const int nstripe = (int)((dm / E + kWave - 1) / kWave);
    const int64_t nblk = std::min<int64_t>(kStripeBlocks, (rows + kWaves - 1) / kWaves);
    if (rows > 0) {
      HDCM_CHECK_ARG(y_row_stride >= dm && gate_row_stride >= dm && dout_row_stride >= dm && dy_row_stride >= dm &&
                         dgate_row_stride >= dm,
                     HDCM_EINVAL);
      HDCM_CHECK_ARG(y_row_stride % E == 0 && gate_row_stride % E == 0 && dout_row_stride % E == 0 &&
                         dy_row_stride % E == 0 && dgate_row_stride % E == 0 && hdcm_aligned16(y) &&
                         hdcm_aligned16(gate) && hdcm_aligned16(dout) && hdcm_aligned16(dy) && hdcm_aligned16(dgate) &&
                         hdcm_aligned16(gn_w) && hdcm_aligned16(gn_b),
                     HDCM_EALIGN);
      const dim3 grid((unsigned)(nblk * nstripe));
#define HDCM_GNS_CASE(TT, HDV)                                                                                      \
  if (hd == HDV) {                                                                                                  \
    HDCM_LAUNCH((gnorm_gate_bwd_rows_kernel<TT, HDV>), grid, dim3(kThreads), 0, s, (const TT*)y,            \
                       y_row_stride, (const TT*)gate, gate_row_stride, (const TT*)gn_w, (const TT*)gn_b, eps,       \
                       (const TT*)dout, dout_row_stride, (TT*)dy, dy_row_stride, (TT*)dgate, dgate_row_stride,      \
                       (float*)ws, rows, (int)dm, nstripe);                                                         \
  }
      if (dtype == HDCM_F32) {
        HDCM_GNS_CASE(float, 16) HDCM_GNS_CASE(float, 32) HDCM_GNS_CASE(float, 64) HDCM_GNS_CASE(float, 128)
      } else {
        HDCM_GNS_CASE(bf16_t, 16) HDCM_GNS_CASE(bf16_t, 32) HDCM_GNS_CASE(bf16_t, 64) HDCM_GNS_CASE(bf16_t, 128)
      }
#undef HDCM_GNS_CASE
      const int st = hdcm_launch_status();
      if (st) return st;
    }
    // workgroup m left part[m][2][dm]: d gn_w is the sum of part[m][0], d gn_b of part[m][1]
    return hdcm_colsum((const float*)ws, 2 * dm, rows > 0 ? (int)nblk : 0, 2 * (int)dm, 2 * (int)dm, 0, dgn_w,
                       (int)dm, dgn_b, s);
  }
  const int nwaves = (int)(H * kWavesPerHead);
  if (rows > 0) {
    HDCM_CHECK_ARG(y_row_stride >= dm && gate_row_stride >= dm && dout_row_stride >= dm && dy_row_stride >= dm &&
                       dgate_row_stride >= dm,
                   HDCM_EINVAL);
    const dim3 grid((unsigned)(nwaves / kWaves));
#define HDCM_GNG_CASE(TT, HDV)                                                                                      \
  if (hd == HDV) {                                                                                                  \
    HDCM_LAUNCH((gnorm_gate_bwd_kernel<TT, HDV>), grid, dim3(kThreads), 0, s, (const TT*)y, y_row_stride,     \
                       (const TT*)gate, gate_row_stride, (const TT*)gn_w, (const TT*)gn_b, eps, (const TT*)dout,    \
                       dout_row_stride, (TT*)dy, dy_row_stride, (TT*)dgate, dgate_row_stride, (float*)ws, rows,     \
                       (int)H);                                                                                     \
  }
    if (dtype == HDCM_F32) {
      HDCM_GNG_CASE(float, 16) HDCM_GNG_CASE(float, 32) HDCM_GNG_CASE(float, 48) HDCM_GNG_CASE(float, 64)
      HDCM_GNG_CASE(float, 80) HDCM_GNG_CASE(float, 96) HDCM_GNG_CASE(float, 112) HDCM_GNG_CASE(float, 128)
    } else {
      HDCM_GNG_CASE(bf16_t, 16) HDCM_GNG_CASE(bf16_t, 32) HDCM_GNG_CASE(bf16_t, 48) HDCM_GNG_CASE(bf16_t, 64)
      HDCM_GNG_CASE(bf16_t, 80) HDCM_GNG_CASE(bf16_t, 96) HDCM_GNG_CASE(bf16_t, 112) HDCM_GNG_CASE(bf16_t, 128)
    }
#undef HDCM_GNG_CASE
    const int st = hdcm_launch_status();
    if (st) return st;
  }
  // wave w = h + H m left part[w][2][hd]: column h*hd + i of d gn_w sums part[w][0][i] over m
  // (with no rows the sums are empty: zero gradients)
  const int nk = rows > 0 ? nwaves / (int)H : 0;
  const int64_t kstride = H * 2 * hd;
  const int st = hdcm_colsum((const float*)ws, kstride, nk, (int)dm, (int)hd, 2 * hd, dgn_w, (int)dm, nullptr, s);
  if (st) return st;
  return hdcm_colsum((const float*)ws + hd, kstride, nk, (int)dm, (int)hd, 2 * hd, dgn_b, (int)dm, nullptr, s);
}

extern "C" int hdcm_slot_phi_prep(const void* projs, int64_t proj_row_stride, int64_t q_col, void* z,
                                  int64_t z_row_stride, int64_t rows, int64_t dm, int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG((projs && z) || rows == 0, HDCM_EINVAL);
  HDCM_CHECK_ARG(rows >= 0 && dm > 0 && q_col >= 0, HDCM_EINVAL);
  if (rows == 0) return HDCM_OK;
  const int E = 16 / hdcm_elt_size(dtype);
  HDCM_CHECK_ARG(proj_row_stride >= q_col + 3 * dm && z_row_stride >= 4 * dm, HDCM_EINVAL);
  HDCM_CHECK_ARG(dm % E == 0 && q_col % E == 0 && proj_row_stride % E == 0 && z_row_stride % E == 0 &&
                     hdcm_aligned16(projs) && hdcm_aligned16(z),
                 HDCM_EALIGN);
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(grid_for(rows * (dm / E)));
  if (dtype == HDCM_F32)
    HDCM_LAUNCH((phi_prep_kernel<float>), grid, dim3(kThreads), 0, s, (const float*)projs, proj_row_stride,
                       (int)q_col, (float*)z, z_row_stride, rows, (int)dm);
  else
    HDCM_LAUNCH((phi_prep_kernel<bf16_t>), grid, dim3(kThreads), 0, s, (const bf16_t*)projs, proj_row_stride,
                       (int)q_col, (bf16_t*)z, z_row_stride, rows, (int)dm);
  return hdcm_launch_status();
}

extern "C" int hdcm_slot_phi_chain(const void* projs, int64_t proj_row_stride, int64_t q_col, void* dprojs,
                                   int64_t dprojs_row_stride, int64_t rows, int64_t dm, int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG((projs && dprojs) || rows == 0, HDCM_EINVAL);
  HDCM_CHECK_ARG(rows >= 0 && dm > 0 && q_col >= 0, HDCM_EINVAL);
  if (rows == 0) return HDCM_OK;
  const int E = 16 / hdcm_elt_size(dtype);
  HDCM_CHECK_ARG(proj_row_stride >= q_col + 2 * dm && dprojs_row_stride >= q_col + 2 * dm, HDCM_EINVAL);
  HDCM_CHECK_ARG(dm % E == 0 && q_col % E == 0 && proj_row_stride % E == 0 && dprojs_row_stride % E == 0 &&
                     hdcm_aligned16(projs) && hdcm_aligned16(dprojs),
                 HDCM_EALIGN);
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(grid_for(rows * (2 * dm / E)));
  if (dtype == HDCM_F32)
    HDCM_LAUNCH((phi_chain_kernel<float>), grid, dim3(kThreads), 0, s, (const float*)projs, proj_row_stride,
                       (int)q_col, (float*)dprojs, dprojs_row_stride, rows, (int)dm);
  else
    HDCM_LAUNCH((phi_chain_kernel<bf16_t>), grid, dim3(kThreads), 0, s, (const bf16_t*)projs, proj_row_stride,
                       (int)q_col, (bf16_t*)dprojs, dprojs_row_stride, rows, (int)dm);
  return hdcm_launch_status();
}
