// Recurrent single-token step of the HdcMamba block for gfx950 (prefill -> decode).
//
// A prefill leaves, per block: the last three block-input rows (the conv history), the SSM
// state h [B,ds] and the slot state at a chunk boundary.  Each decode step then advances
// one token per batch row with the same semantics as the chunked forward
// (hdcmamba/model.py:22-72, 175-233, 236-295):
//
//   norm_conv_step:  u = LN(x_t); out = sum_k u_{t-3+k} w_k + b, rows before the sequence
//                    start having u = ln_b (the LayerNorm of a zero row); the history keeps
//                    raw rows and is shifted in place.
//   mixer_step:      SSM      h = exp(dt*A) h + dt*b*x,  y_ssm = h          (fp32 state)
//                    slot     the weight of (t, j) is gamma^(t-j) inside t's chunk and
//                             gamma^(t-j-1) across chunks, so with c = t mod C
//                               S_eff_t = sum_{j in chunk, j<=t} gamma^(t-j) phi(k_j)^T v_j
//                                         + gamma^c S_prev,     y_t = phi(q_t) S_eff_t,
//                             carried as S_eff_t = S_prev + phi(k_t)^T v_t (c = 0) or
//                             gamma S_eff_{t-1} + phi(k_t)^T v_t (c > 0), kept in S_intra
//                             between the tokens of a chunk; at the chunk's last token
//                               S_prev <- S_eff_t + (gamma^C - gamma^(C-1)) S_prev
//                             (= gamma^C S_prev + the chunk's own sum).  A token reads one
//                             fp32 state (two at a chunk's first and last token) and writes one.
//                    then GroupNorm over the head's hd values and the sigmoid gate, written
//                    next to y_ssm in the `combined` row.
//
// Decode is weight- and state-bandwidth bound (the GEMMs around it read every weight once
// per step), so these kernels are simple: one workgroup per batch row (norm_conv_step) and
// one per (head, batch) plus one per batch for the SSM channels (mixer_step).  Head dims
// are the multiples of 16 up to 128.
#include "hdcm_common.h"

using namespace hdcm;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// Sum of N values per thread over the workgroup; every thread receives the totals.
template <int N>
__device__ __forceinline__ void block_sum(float (&v)[N], float* red) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
#pragma unroll
  for (int n = 0; n < N; ++n) v[n] = wave_sum(v[n]);
  __syncthreads();
  if (lane == 0) {
#pragma unroll
    for (int n = 0; n < N; ++n) red[w * N + n] = v[n];
  }
  __syncthreads();
#pragma unroll
  for (int n = 0; n < N; ++n) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) s += red[k * N + n];
    v[n] = s;
  }
}

// One workgroup per batch row; thread t owns 16-byte column groups t, t+256, ...
template <typename T, int NG>
__global__ __launch_bounds__(kThreads) void norm_conv_step_kernel(
    const T* __restrict__ x, int64_t x_rs, const T* __restrict__ ln_w, const T* __restrict__ ln_b,
    const T* __restrict__ conv_w, const T* __restrict__ conv_b, T* __restrict__ hist,
    T* __restrict__ out, int64_t o_rs, int D, float eps) {
  constexpr int E = Vec<T>::N;
  __shared__ float red[kWaves * 8];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int G = D / E;
  // rows 0..2: history (oldest first), row 3: the new token
  const T* rows[4] = {hist + ((int64_t)b * 3 + 0) * D, hist + ((int64_t)b * 3 + 1) * D,
                      hist + ((int64_t)b * 3 + 2) * D, x + (int64_t)b * x_rs};
  // Every load of the step is issued up front: the four rows, then the LayerNorm and conv
  // parameters (kept as stored until after the statistics), so one memory round trip
  // covers the whole step.  Groups past G read group 0 (their results are not stored).
  uint4 raw[4][NG], prm[7][NG];
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int g = tid + kThreads * i < G ? tid + kThreads * i : 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) raw[k][i] = ldg16(rows[k] + g * E);
  }
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int g = tid + kThreads * i < G ? tid + kThreads * i : 0;
    prm[0][i] = ldg16(ln_w + g * E);
    prm[1][i] = ldg16(ln_b + g * E);
    prm[2][i] = ldg16(conv_b + g * E);
#pragma unroll
    for (int k = 0; k < 4; ++k) prm[3 + k][i] = ldg16(conv_w + (int64_t)g * E * 4 + k * E);
  }
  float r[4][NG][E];
  float st[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) st[n] = 0.f;
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const bool ok = tid + kThreads * i < G;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      unpack16<T>(raw[k][i], r[k][i]);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float v = ok ? r[k][i][e] : 0.f;
        st[2 * k] += v;
        st[2 * k + 1] += v * v;
      }
    }
  }
  block_sum<8>(st, red);
  float mean[4], rstd[4];
  const float invD = 1.0f / (float)D;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    mean[k] = st[2 * k] * invD;
    const float var = fmaxf(st[2 * k + 1] * invD - mean[k] * mean[k], 0.f);
    rstd[k] = rsqrtf(var + eps);
  }
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int g = tid + kThreads * i;
    if (g >= G) continue;
    float w[E], bb[E], cb[E], cw[4 * E], o[E];
    unpack16<T>(prm[0][i], w);
    unpack16<T>(prm[1][i], bb);
    unpack16<T>(prm[2][i], cb);
#pragma unroll
    for (int k = 0; k < 4; ++k) unpack16<T>(prm[3 + k][i], cw + k * E);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float acc = cb[e];
#pragma unroll
      for (int k = 0; k < 4; ++k) acc += ((r[k][i][e] - mean[k]) * rstd[k] * w[e] + bb[e]) * cw[4 * e + k];
      o[e] = acc;
    }
    store16<T>(out + (int64_t)b * o_rs + g * E, o);
    // shift the history: rows 1, 2 and the new token become rows 0, 1, 2
#pragma unroll
    for (int k = 0; k < 3; ++k) *reinterpret_cast<uint4*>(hist + ((int64_t)b * 3 + k) * D + g * E) = raw[k + 1][i];
  }
}


// grid (H + 1, B): x < H is head x's slot step, x == H the SSM channels of batch row b.
// A slot workgroup owns one head's two fp32 states [HD][HD]; thread t holds 4 consecutive
// columns (float4) of rows t / CG + RGS * k, so every state load of the step is issued
// before the first use and the row sums of y are finished through LDS.
template <typename T, int HD>
__global__ __launch_bounds__(kThreads) void mixer_step_kernel(
    const T* __restrict__ projs, int64_t prs, int q_col, int dm, const T* __restrict__ gamma,
    float* __restrict__ S_prev, float* __restrict__ S_intra, int c_arg, const int* __restrict__ c_dev, int C,
    const T* __restrict__ gn_w,
    const T* __restrict__ gn_b, float gn_eps, const T* __restrict__ A_log, float* __restrict__ hs,
    int ds, T* __restrict__ out, int64_t ors, int y_col, int g_col) {
  constexpr int CG = HD / 4;              // float4 column groups of a state row
  constexpr int RGS = kThreads / CG;      // row groups
  constexpr int RPT = (HD + RGS - 1) / RGS;  // rows per thread
  __shared__ float sq[HD], sk[HD], sv[HD];
  __shared__ float sy[RGS][HD + 4];
  __shared__ float red[kWaves * 2];
  const int tid = threadIdx.x, b = blockIdx.y, H = gridDim.x - 1;
  const T* row = projs + (int64_t)b * prs;
  T* orow = out + (int64_t)b * ors;

  if ((int)blockIdx.x == H) {  // SSM: h = exp(dt*A) h + dt*b*x
    for (int ch = tid; ch < ds; ch += kThreads) {
      const float dt = softplus20(to_f<T>(row[ch]));
      const float a = fexp(-dt * fexp(to_f<T>(A_log[ch])));
      const float u = dt * to_f<T>(row[2 * ds + ch]) * to_f<T>(row[ds + ch]);
      float* hp = hs + (int64_t)b * ds + ch;
      const float h = a * *hp + u;
      *hp = h;
      orow[y_col + ch] = from_f<T>(h);
    }
    return;
  }

  const int h = blockIdx.x;
  const int cgi = tid % CG, rg = tid / CG;
  const bool act = rg < RGS;
  const int64_t sbase = (((int64_t)b * H + h) * HD) * HD + 4 * cgi;
  // chunk offset: from device memory when the step runs inside a captured graph
  const int c = c_dev != nullptr ? __builtin_amdgcn_readfirstlane(*c_dev) : c_arg;
  // This token's q, k, v (needed first, for the LDS vectors), its gate and the GroupNorm
  // affine go out ahead of the states and are converted only after the state loads are
  // issued, so the wait for them overlaps the states' round trip.  Branch-free at a clamped
  // column (threads past HD load column HD-1 and do not use it).
  const T* q = row + q_col + h * HD;
  const int hc = min(tid, HD - 1);
  const T q_raw = q[hc], k_raw = q[dm + hc], v_raw = q[2 * dm + hc];
  const T gate_raw = row[q_col + 3 * dm + h * HD + hc], gnw_raw = gn_w[h * HD + hc], gnb_raw = gn_b[h * HD + hc];
  const T gamma_raw = gamma[h];
  // The state the token builds on: the previous token's S_eff kept in S_intra, loaded while
  // the offset is still in flight (right for every token but a chunk's first), or S_prev at a
  // chunk's first token; S_prev again at a chunk's last token, where it is folded into the
  // next boundary state.
  float4 sz[RPT], sp[RPT];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int i = rg + RGS * k;
    if (act && i < HD) sz[k] = *reinterpret_cast<const float4*>(S_intra + sbase + (int64_t)i * HD);
  }
  const bool first = c == 0, last = c == C - 1;
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int i = rg + RGS * k;
    if (act && i < HD) {
      if (first) sz[k] = *reinterpret_cast<const float4*>(S_prev + sbase + (int64_t)i * HD);
      else if (last) sp[k] = *reinterpret_cast<const float4*>(S_prev + sbase + (int64_t)i * HD);
    }
  }
  const float g = to_f<T>(gamma_raw);
  const float lg2 = log2f(g);
  if (tid < HD) {
    // phi(q), phi(k) rounded to the activation dtype as in the chunked kernels' operands
    sq[tid] = rnd<T>(phi_f(to_f<T>(q_raw)));
    sk[tid] = rnd<T>(phi_f(to_f<T>(k_raw)));
    sv[tid] = to_f<T>(v_raw);
  }
  __syncthreads();

  // S_eff = gz * Z + phi(k)^T v with gz = 1 at a chunk's first token (Z = S_prev) and gamma
  // after it (Z = the previous token's S_eff = S_intra + gamma^(c-1) S_prev); y = phi(q) S_eff.
  // At the chunk's last token the boundary state gamma^C S_prev + S_intra is
  // S_eff + (gamma^C - gamma^(C-1)) S_prev.
  const float gz = first ? 1.0f : g;
  const float dC = fexp2((float)C * lg2) - fexp2((float)(C - 1) * lg2);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (act) {
    const float v4[4] = {sv[4 * cgi], sv[4 * cgi + 1], sv[4 * cgi + 2], sv[4 * cgi + 3]};
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int i = rg + RGS * k;
      if (i >= HD) continue;
      const float ki = sk[i], qi = sq[i];
      const float z[4] = {sz[k].x, sz[k].y, sz[k].z, sz[k].w};
      float n[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        n[e] = fmaf(gz, z[e], ki * v4[e]);
        acc[e] = fmaf(qi, n[e], acc[e]);
      }
      const int64_t off = sbase + (int64_t)i * HD;
      if (last) {
        const float4 po = first ? sz[k] : sp[k];
        *reinterpret_cast<float4*>(S_prev + off) =
            make_float4(fmaf(dC, po.x, n[0]), fmaf(dC, po.y, n[1]), fmaf(dC, po.z, n[2]), fmaf(dC, po.w, n[3]));
      } else {
        *reinterpret_cast<float4*>(S_intra + off) = make_float4(n[0], n[1], n[2], n[3]);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) sy[rg][4 * cgi + e] = acc[e];
  }
  __syncthreads();
  float y = 0.f;
  if (tid < HD) {
#pragma unroll
    for (int k = 0; k < RGS; ++k) y += sy[k][tid];
  }
  // GroupNorm over the head's hd values, then the gate.  Up to 64 values they are all in wave 0,
  // whose own sums are the workgroup's (the other waves add zeros), so the other waves are done
  // and no barrier is needed.
  float st[2] = {tid < HD ? y : 0.f, tid < HD ? y * y : 0.f};
  if constexpr (HD <= kWave) {
    if (tid >= kWave) return;
    st[0] = wave_sum(st[0]);
    st[1] = wave_sum(st[1]);
  } else {
    block_sum<2>(st, red);
  }
  const float mean = st[0] / (float)HD;
  const float var = fmaxf(st[1] / (float)HD - mean * mean, 0.f);
  const float rinv = rsqrtf(var + gn_eps);
  if (tid < HD) {
    const int col = h * HD + tid;
    const float gate = to_f<T>(gate_raw);
    const float yn = (y - mean) * rinv * to_f<T>(gnw_raw) + to_f<T>(gnb_raw);
    orow[g_col + col] = from_f<T>(yn * frcp(1.0f + fexp(-gate)));
  }
}

__global__ void chunk_pos_advance_kernel(int* pos, int C) {
  if (threadIdx.x == 0) {
    const int p = *pos + 1;
    *pos = p == C ? 0 : p;
  }
}

template <typename T>
int launch_norm_conv_step(const void* x, int64_t x_rs, const void* ln_w, const void* ln_b,
                          const void* conv_w, const void* conv_b, void* hist, void* out, int64_t o_rs,
                          int64_t B, int64_t D, float eps, hipStream_t s) {
  constexpr int E = Vec<T>::N;
  const int64_t G = D / E;
  const int ng = (int)((G + kThreads - 1) / kThreads);
#define HDCM_NCS_CASE(N)                                                                             \
  if (ng == N) {                                                                                     \
    HDCM_LAUNCH((norm_conv_step_kernel<T, N>), dim3((unsigned)B), dim3(kThreads), 0, s,      \
                       (const T*)x, x_rs, (const T*)ln_w, (const T*)ln_b, (const T*)conv_w,          \
                       (const T*)conv_b, (T*)hist, (T*)out, o_rs, (int)D, eps);                      \
    return hdcm_launch_status();                                                                     \
  }
  HDCM_NCS_CASE(1)
  HDCM_NCS_CASE(2)
  HDCM_NCS_CASE(3)
  HDCM_NCS_CASE(4)
#undef HDCM_NCS_CASE
  return HDCM_EUNSUPPORTED;
}

}  // namespace

extern "C" int hdcm_norm_conv_step_fwd(const void* x, int64_t x_row_stride, const void* ln_w,
                                       const void* ln_b, const void* conv_w, const void* conv_b,
                                       void* hist, void* out, int64_t out_row_stride, int64_t B,
                                       int64_t D, float eps, int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(ln_w && ln_b && conv_w && conv_b && ((x && hist && out) || B == 0), HDCM_EINVAL);
  HDCM_CHECK_ARG(B >= 0 && D > 0 && x_row_stride >= D && out_row_stride >= D, HDCM_EINVAL);
  const int E = 16 / hdcm_elt_size(dtype);
  HDCM_CHECK_ARG(D % E == 0 && x_row_stride % E == 0 && out_row_stride % E == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(hdcm_aligned16(x) && hdcm_aligned16(out) && hdcm_aligned16(hist) && hdcm_aligned16(ln_w) &&
                     hdcm_aligned16(ln_b) && hdcm_aligned16(conv_w) && hdcm_aligned16(conv_b),
                 HDCM_EALIGN);
  HDCM_CHECK_ARG(D / E <= 4 * kThreads && B <= 65535, HDCM_EUNSUPPORTED);
  if (B == 0) return HDCM_OK;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HDCM_F32)
    return launch_norm_conv_step<float>(x, x_row_stride, ln_w, ln_b, conv_w, conv_b, hist, out,
                                        out_row_stride, B, D, eps, s);
  return launch_norm_conv_step<bf16_t>(x, x_row_stride, ln_w, ln_b, conv_w, conv_b, hist, out,
                                       out_row_stride, B, D, eps, s);
}

extern "C" int hdcm_mixer_step_fwd(const void* projs, int64_t proj_row_stride, int64_t q_col,
                                   const void* A_log, float* h, const void* gamma, float* S_prev,
                                   float* S_intra, int64_t pos, const int32_t* pos_dev, int64_t C,
                                   const void* gn_w,
                                   const void* gn_b, float gn_eps, void* out, int64_t out_row_stride,
                                   int64_t y_col, int64_t g_col, int64_t B, int64_t dm, int64_t ds,
                                   int64_t H, int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(A_log && gamma && gn_w && gn_b && ((projs && h && S_prev && S_intra && out) || B == 0),
                 HDCM_EINVAL);
  HDCM_CHECK_ARG(B >= 0 && dm > 0 && ds > 0 && H > 0 && dm % H == 0 && C > 0, HDCM_EINVAL);
  HDCM_CHECK_ARG(pos >= 0 && pos < C, HDCM_EINVAL);
  HDCM_CHECK_ARG(q_col >= 3 * ds && proj_row_stride >= q_col + 4 * dm, HDCM_EINVAL);
  HDCM_CHECK_ARG(y_col >= 0 && g_col >= 0 && out_row_stride >= y_col + ds && out_row_stride >= g_col + dm,
                 HDCM_EINVAL);
  const int64_t hd = dm / H;
  HDCM_CHECK_ARG(hd >= 16 && hd <= 128 && hd % 16 == 0 && H < 65535 && B <= 65535 &&
                     proj_row_stride < ((int64_t)1 << 31),
                 HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(C < ((int64_t)1 << 24), HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(hdcm_aligned16(S_prev) && hdcm_aligned16(S_intra), HDCM_EALIGN);
  if (B == 0) return HDCM_OK;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)(H + 1), (unsigned)B);
#define HDCM_MIX_CASE(TT, HDV)                                                                              \
  if (hd == HDV) {                                                                                           \
    HDCM_LAUNCH((mixer_step_kernel<TT, HDV>), grid, dim3(kThreads), 0, s, (const TT*)projs,          \
                       proj_row_stride, (int)q_col, (int)dm, (const TT*)gamma, S_prev, S_intra, (int)pos,    \
                       (const int*)pos_dev, (int)C, (const TT*)gn_w, (const TT*)gn_b, gn_eps,               \
                       (const TT*)A_log, h, (int)ds, (TT*)out, out_row_stride, (int)y_col, (int)g_col);      \
    return hdcm_launch_status();                                                                             \
  }
  if (dtype == HDCM_F32) {
    HDCM_MIX_CASE(float, 16)
    HDCM_MIX_CASE(float, 32)
    HDCM_MIX_CASE(float, 48)
    HDCM_MIX_CASE(float, 64)
    HDCM_MIX_CASE(float, 80)
    HDCM_MIX_CASE(float, 96)
    HDCM_MIX_CASE(float, 112)
    HDCM_MIX_CASE(float, 128)
  } else {
    HDCM_MIX_CASE(bf16_t, 16)
    HDCM_MIX_CASE(bf16_t, 32)
    HDCM_MIX_CASE(bf16_t, 48)
    HDCM_MIX_CASE(bf16_t, 64)
    HDCM_MIX_CASE(bf16_t, 80)
    HDCM_MIX_CASE(bf16_t, 96)
    HDCM_MIX_CASE(bf16_t, 112)
    HDCM_MIX_CASE(bf16_t, 128)
  }
#undef HDCM_MIX_CASE
  return HDCM_EUNSUPPORTED;
}

extern "C" int hdcm_chunk_pos_advance(int32_t* pos_dev, int64_t C, void* stream) {
  HDCM_CHECK_ARG(pos_dev != nullptr && C > 0 && C < ((int64_t)1 << 24), HDCM_EINVAL);
  HDCM_LAUNCH(chunk_pos_advance_kernel, dim3(1), dim3(kWave), 0, (hipStream_t)stream, (int*)pos_dev,
                     (int)C);
  return hdcm_launch_status();
}
