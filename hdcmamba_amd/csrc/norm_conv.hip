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
// which makes the t<0 halo exactly xhat = 0.  Raw rows are prefetched 4 rows ahead so
// several 128-bit loads per lane are in flight while the current rows are reduced.
//
// The kernel is bound by its per-row instruction stream, not by HBM: inside the model a plain
// copy of the same rows at the same point takes two thirds of its time.  So a full run is
// straight-line code with no per-row checks, rows go in pairs so the two rows' reductions
// (DPP moves within 16-lane rows, then v_permlane16_swap/v_permlane32_swap across them)
// interleave instead of each waiting out its own hazards, bf16 row sums come from
// v_dot2_f32_bf16 on the packed words, lane masks exist only when D is not a multiple of
// 64 column groups, and each output is one chain of 4 FMAs.  The sequence's last, partial
// run, and every run of rows wider than 32 columns per lane, takes rows one at a time.
//
// Measured alternatives that ran slower or no faster inside the model's forward: two waves
// per row with Chan-merged half-row statistics (higher occupancy, one barrier per row),
// numbering blocks so that each XCD walks a contiguous range of rows, 32-row runs, a deeper
// prefetch, and the 3-row halo handed from wave to wave through LDS (the halo re-read hits
// the caches).
#include "hdcm_common.h"

using namespace hdcm;

namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kPF = 4;  // prefetch distance (rows): two row pairs

// One row's 16-byte groups; MASK: groups past D (G groups) read as zeros.
template <typename T, int NG, bool MASK>
__device__ __forceinline__ void load_row(uint4 (&raw)[NG], const T* row, int lane, int G) {
  constexpr int E = Vec<T>::N;
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int g = lane + kWave * i;
    raw[i] = (!MASK || g < G) ? ldg16(row + (int64_t)g * E) : make_uint4(0, 0, 0, 0);
  }
}

// This lane's part of a row sum, from the raw words: bf16 pairs through v_dot2_f32_bf16
// against (1, 1), so the sum does not wait for the unpacking.  Lanes past D hold zeros.
template <typename T, int NG>
__device__ __forceinline__ float lane_sum(const uint4 (&raw)[NG]) {
  float s = 0.f;
  if constexpr (sizeof(T) == 2) {
    typedef __bf16 b16x2 __attribute__((ext_vector_type(2)));
    const b16x2 one = __builtin_bit_cast(b16x2, 0x3f803f80u);
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const uint32_t w[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b16x2, w[k]), one, s, false);
    }
  } else {
#pragma unroll
    for (int i = 0; i < NG; ++i)
      s += (__uint_as_float(raw[i].x) + __uint_as_float(raw[i].y)) +
           (__uint_as_float(raw[i].z) + __uint_as_float(raw[i].w));
  }
  return s;
}

template <int C, int RM, int NR>
__device__ __forceinline__ void dpp_add(float (&v)[NR]) {
#pragma unroll
  for (int n = 0; n < NR; ++n)
    v[n] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[n]), C, RM, 0xf, false));
}

// Sums over the wave of NR values at once, their chains interleaved: DPP moves within each
// 16-lane row, then the gfx950 row swaps (v_permlane16_swap, v_permlane32_swap) across rows,
// which leave the total in every lane.
template <int NR>
__device__ __forceinline__ void wave_totals(float (&v)[NR]) {
  dpp_add<0xB1, 0xf>(v);   // quad [1,0,3,2]
  dpp_add<0x4E, 0xf>(v);   // quad [2,3,0,1]
  dpp_add<0x141, 0xf>(v);  // row_half_mirror
  dpp_add<0x140, 0xf>(v);  // row_mirror
#pragma unroll
  for (int n = 0; n < NR; ++n) v[n] = quad_group_sum(v[n]);
}

// Normalise NR rows in registers: xh = (x - mean) * rstd with the centred (two-pass) biased
// variance.  MASK: D is not a multiple of the wave's 64 column groups, and lanes past D must
// hold 0.
template <typename T, int NG, int NR, bool MASK>
__device__ __forceinline__ void ln_rows(const uint4 (&raw)[NR][NG], float (&xh)[NR][NG][Vec<T>::N],
                                        int lane, int G, float invD, float eps) {
  constexpr int E = Vec<T>::N;
  float s[NR], q[NR];
#pragma unroll
  for (int n = 0; n < NR; ++n) s[n] = lane_sum<T, NG>(raw[n]);
  wave_totals<NR>(s);
#pragma unroll
  for (int n = 0; n < NR; ++n) {
    const float mean = s[n] * invD;
    float qa = 0.f, qb = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const bool ok = !MASK || (lane + kWave * i) < G;
      unpack16<T>(raw[n][i], xh[n][i]);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float c = ok ? xh[n][i][e] - mean : 0.f;
        xh[n][i][e] = c;
        if (e & 1) qb = fmaf(c, c, qb);
        else qa = fmaf(c, c, qa);
      }
    }
    q[n] = qa + qb;
  }
  wave_totals<NR>(q);
#pragma unroll
  for (int n = 0; n < NR; ++n) {
    const float rstd = rsqrtf(q[n] * invD + eps);
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int e = 0; e < Vec<T>::N; ++e) xh[n][i][e] *= rstd;
  }
}

// out[t] = sum_k (w*c_k) * xhat[t-3+k] + bt for one row, stored as 16-byte groups.
template <typename T, int NG, bool MASK>
__device__ __forceinline__ void conv_store(T* orow, const float (&wc)[4][NG][Vec<T>::N],
                                           const float (&bt)[NG][Vec<T>::N], const float (&h3)[NG][Vec<T>::N],
                                           const float (&h2)[NG][Vec<T>::N], const float (&h1)[NG][Vec<T>::N],
                                           const float (&h0)[NG][Vec<T>::N], int lane, int G) {
  constexpr int E = Vec<T>::N;
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int g = lane + kWave * i;
    float o[E];
#pragma unroll
    for (int e = 0; e < E; ++e)
      o[e] = fmaf(wc[3][i][e], h0[i][e],
                  fmaf(wc[2][i][e], h1[i][e], fmaf(wc[1][i][e], h2[i][e], fmaf(wc[0][i][e], h3[i][e], bt[i][e]))));
    if (!MASK || g < G) store16<T>(orow + (int64_t)g * E, o);
  }
}

template <typename T, int NG, int kRows, bool MASK>
__global__ __launch_bounds__(kWavesPerBlock* kWave) void norm_conv_kernel(
    const T* __restrict__ x, int64_t x_bs, int64_t x_rs, const T* __restrict__ ln_w,
    const T* __restrict__ ln_b, const T* __restrict__ conv_w, const T* __restrict__ conv_b,
    T* __restrict__ out, int64_t o_bs, int64_t o_rs, int L, int D, float eps) {
  static_assert(kRows % 2 == 0 && kPF % 2 == 0, "rows are taken in pairs");
  constexpr int E = Vec<T>::N;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t t0 = ((int64_t)blockIdx.x * kWavesPerBlock + wave) * kRows;
  if (t0 >= L) return;
  const int G = D / E;
  const float invD = 1.0f / (float)D;
  const T* xb = x + (int64_t)blockIdx.y * x_bs;
  T* ob = out + (int64_t)blockIdx.y * o_bs;

  // Up to 32 columns per lane a full run takes the straight-line path; wider rows do not fit
  // its registers and go one row at a time.
  constexpr bool kFast = NG * E <= 32;
  // Up to 16 columns per lane the raw parameters fit in registers beside the rows in flight,
  // so every load of the prologue is issued before the first wait: the LayerNorm and conv
  // parameters (oldest, so folding them waits for nothing else), the history rows t0-3 ..
  // t0-1, then the prefetch ring of a full run.  Wider rows issue the ring, then load and fold
  // the parameters, then load the history rows.
  constexpr bool kEarly = NG * E <= 16;
  const bool full = kFast && t0 + kRows <= L;  // rows t0 .. t0+kRows-1 all exist
  // Folded parameters: wc[k] = ln_w * conv_w[:,k], bt = ln_b * sum_k conv_w[:,k] + conv_b.
  // prm: ln_w, ln_b, conv_b, then the 4 tap groups of conv_w ([D,4]) of a group, as stored.
  float wc[4][NG][E], bt[NG][E];
  auto load_group = [&](int i, uint4 (&prm)[7]) __attribute__((always_inline)) {
    const int g = lane + kWave * i;
    const int gs = g < G ? g : 0;  // groups past D read group 0; zeroed at the fold
    prm[0] = ldg16(ln_w + gs * E);
    prm[1] = ldg16(ln_b + gs * E);
    prm[2] = ldg16(conv_b + gs * E);
#pragma unroll
    for (int k = 0; k < 4; ++k) prm[3 + k] = ldg16(conv_w + (int64_t)gs * E * 4 + k * E);
  };
  auto fold_group = [&](int i, const uint4 (&prm)[7]) __attribute__((always_inline)) {
    const bool ok = lane + kWave * i < G;
    float w[E], bb[E], cb[E], cw[4 * E];
    unpack16<T>(prm[0], w);
    unpack16<T>(prm[1], bb);
    unpack16<T>(prm[2], cb);
#pragma unroll
    for (int k = 0; k < 4; ++k) unpack16<T>(prm[3 + k], cw + k * E);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      // conv_w is [D,4]: column c = g*E+e has taps cw[4e..4e+3].
      const float c0 = ok ? cw[4 * e + 0] : 0.f, c1 = ok ? cw[4 * e + 1] : 0.f;
      const float c2 = ok ? cw[4 * e + 2] : 0.f, c3 = ok ? cw[4 * e + 3] : 0.f;
      const float we = ok ? w[e] : 0.f, be = ok ? bb[e] : 0.f, ce = ok ? cb[e] : 0.f;
      wc[0][i][e] = we * c0;
      wc[1][i][e] = we * c1;
      wc[2][i][e] = we * c2;
      wc[3][i][e] = we * c3;
      bt[i][e] = be * (c0 + c1 + c2 + c3) + ce;
    }
  };
  uint4 hr[3][NG];
  auto load_hist = [&]() __attribute__((always_inline)) {
    load_row<T, NG, MASK>(hr[0], xb + (t0 >= 3 ? (t0 - 3) : 0) * x_rs, lane, G);
    load_row<T, NG, MASK>(hr[1], xb + (t0 >= 2 ? (t0 - 2) : 0) * x_rs, lane, G);
    load_row<T, NG, MASK>(hr[2], xb + (t0 >= 1 ? (t0 - 1) : 0) * x_rs, lane, G);
  };
  uint4 ring[kPF][NG];
  auto load_ring = [&]() __attribute__((always_inline)) {
    if (full) {
#pragma unroll
      for (int p = 0; p < kPF; ++p) load_row<T, NG, MASK>(ring[p], xb + (t0 + p) * x_rs, lane, G);
    }
  };
  if constexpr (kEarly) {
    uint4 prm[NG][7];
#pragma unroll
    for (int i = 0; i < NG; ++i) load_group(i, prm[i]);
    load_hist();
    load_ring();
#pragma unroll
    for (int i = 0; i < NG; ++i) fold_group(i, prm[i]);
  } else {
    load_ring();
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      uint4 prm[7];
      load_group(i, prm);
      fold_group(i, prm);
    }
    load_hist();
  }

  // History rows t0-3, t0-2, t0-1 (xhat = 0 before the sequence start).
  float h3[NG][E], h2[NG][E], h1[NG][E];
  {
    float hx[3][NG][E];
    ln_rows<T, NG, 3, MASK>(hr, hx, lane, G, invD, eps);
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        h3[i][e] = t0 < 3 ? 0.f : hx[0][i][e];
        h2[i][e] = t0 < 2 ? 0.f : hx[1][i][e];
        h1[i][e] = t0 < 1 ? 0.f : hx[2][i][e];
      }
  }

  if constexpr (kFast) if (full) {
    // A full run: straight-line code, rows in pairs so the two rows' reductions interleave.
#pragma unroll
    for (int r = 0; r < kRows; r += 2) {
      uint4 cur[2][NG];
#pragma unroll
      for (int i = 0; i < NG; ++i) {
        cur[0][i] = ring[r % kPF][i];
        cur[1][i] = ring[(r + 1) % kPF][i];
      }
      if (r + kPF < kRows) load_row<T, NG, MASK>(ring[r % kPF], xb + (t0 + r + kPF) * x_rs, lane, G);
      if (r + 1 + kPF < kRows) load_row<T, NG, MASK>(ring[(r + 1) % kPF], xb + (t0 + r + 1 + kPF) * x_rs, lane, G);
      float xc[2][NG][E];
      ln_rows<T, NG, 2, MASK>(cur, xc, lane, G, invD, eps);
      conv_store<T, NG, MASK>(ob + (t0 + r) * o_rs, wc, bt, h3, h2, h1, xc[0], lane, G);
      conv_store<T, NG, MASK>(ob + (t0 + r + 1) * o_rs, wc, bt, h2, h1, xc[0], xc[1], lane, G);
#pragma unroll
      for (int i = 0; i < NG; ++i)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          h3[i][e] = h1[i][e];
          h2[i][e] = xc[0][i][e];
          h1[i][e] = xc[1][i][e];
        }
    }
    return;
  }
  // The sequence's last, partial run (and every run of wide rows): one row at a time, loaded
  // when it is needed.
  const int64_t t_end = t0 + kRows < L ? t0 + kRows : L;
#pragma unroll 1
  for (int64_t t = t0; t < t_end; ++t) {
    uint4 cur[1][NG];
    load_row<T, NG, MASK>(cur[0], xb + t * x_rs, lane, G);
    float xc[1][NG][E];
    ln_rows<T, NG, 1, MASK>(cur, xc, lane, G, invD, eps);
    conv_store<T, NG, MASK>(ob + t * o_rs, wc, bt, h3, h2, h1, xc[0], lane, G);
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        h3[i][e] = h2[i][e];
        h2[i][e] = h1[i][e];
        h1[i][e] = xc[0][i][e];
      }
  }
}

template <typename T, int NG, int kRows>
void launch_rows(const void* x, int64_t x_bs, int64_t x_rs, const void* ln_w, const void* ln_b,
                 const void* conv_w, const void* conv_b, void* out, int64_t o_bs, int64_t o_rs,
                 int64_t B, int64_t L, int64_t D, float eps, hipStream_t s) {
  const int64_t rows_per_block = (int64_t)kWavesPerBlock * kRows;
  dim3 grid((unsigned)((L + rows_per_block - 1) / rows_per_block), (unsigned)B);
  if (D / Vec<T>::N == NG * kWave)
    HDCM_LAUNCH((norm_conv_kernel<T, NG, kRows, false>), grid, dim3(kWavesPerBlock * kWave), 0, s,
                (const T*)x, x_bs, x_rs, (const T*)ln_w, (const T*)ln_b, (const T*)conv_w,
                (const T*)conv_b, (T*)out, o_bs, o_rs, (int)L, (int)D, eps);
  else
    HDCM_LAUNCH((norm_conv_kernel<T, NG, kRows, true>), grid, dim3(kWavesPerBlock * kWave), 0, s,
                (const T*)x, x_bs, x_rs, (const T*)ln_w, (const T*)ln_b, (const T*)conv_w,
                (const T*)conv_b, (T*)out, o_bs, o_rs, (int)L, (int)D, eps);
}

// 16 rows per wave: the 3-row halo is re-read for every 16 rows.
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
  // data pointers of empty inputs (B or L zero) may be NULL
  HDCM_CHECK_ARG(ln_w && ln_b && conv_w && conv_b && ((x && out) || B == 0 || L == 0), HDCM_EINVAL);
  HDCM_CHECK_ARG(B >= 0 && L >= 0 && D > 0, HDCM_EINVAL);
  const int esz = hdcm_elt_size(dtype);
  const int E = 16 / esz;
  HDCM_CHECK_ARG(D % E == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(D / E <= 12 * kWave, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(B <= 65535 && L < (int64_t)1 << 30, HDCM_EUNSUPPORTED);
  if (B == 0 || L == 0) return HDCM_OK;  // nothing is addressed: strides are not checked
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
