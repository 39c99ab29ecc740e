// Tiled bf16 GEMM for gfx950 with fused epilogues:
//   out[t, o] = epi( sum_k X[t, k] W[o, k] ),  X [M, K] rows (tokens), W [N, K] an nn.Linear
// weight (K contiguous in both), fp32 accumulation, one rounding to bf16 at the end.
//   EPI_BIAS:   + bias[o]                                  (in_proj: hdcmamba/model.py:313,340)
//   EPI_ROWLN:  res[t, o] + r_t * (acc - mu_t * s_o)       (out_proj over the row LayerNorm
//               and the residual add: model.py:382-383,394)
//   EPI_ROWSTATS: the same value, with mu_t, r_t from row statistics its producers wrote and s
//               from a cached weight-row-sum vector (see "Row statistics from the producers")
// The row LayerNorm of out_proj's input (no affine, eps) folds into the epilogue:
//   LN(c)_t W^T = r_t (c_t - mu_t 1) W^T = r_t (c_t W^T - mu_t s),  s_o = sum_k W[o, k],
// so the normalized rows never exist in memory.  mu_t, r_t = 1/sqrt(var_t + eps) and s_o
// all come from the operands on their way through the MFMAs: X's rows pass through the B
// fragments in full (K is the row width) and W's rows through the A fragments, and the
// waves add sum c, sum c^2 and sum w with v_dot2_f32_bf16 (against ones, and c against
// itself) while the MFMAs run, each wave taking a quarter or a half of the fragments.
//
// Tiling: a workgroup of 8 waves (two per SIMD, so one wave's MFMAs cover the other's LDS
// reads) computes a 256 (o) x 256 (t) tile; wave w owns 128 o x 64 t ((w & 1), (w >> 1)) as
// 8 x 4 tiles of v_mfma_f32_16x16x32_bf16 with W as the MFMA A operand and X as B, so lane l
// holds outputs of token l % 16 and four consecutive features 4 (l / 16) .. +3 (one 8-byte
// store).  K advances 64 at a time through two LDS buffers filled by direct-to-LDS buffer
// loads (buffer_load_dwordx4 ... lds): while tile k feeds the MFMAs, tile k+1 streams into
// the other buffer; one barrier per K step.  Each load instruction of a wave fills 8 rows
// x 128 bytes; in LDS the 16-byte chunk c of row r sits at chunk c ^ (r & 7), so the
// fragment reads of lanes 0..7 (rows r..r+7, one chunk) fall in eight different bank
// groups (SQ_LDS_BANK_CONFLICT reads 0).  Rows past M or N read as zeros (buffer range
// checking); K columns past K get an out-of-range offset, also zeros.
//
// Row statistics from the producers (EPI_ROWSTATS): the kernels that write the rows of X
// (the scan and the slot gate) also write, per row, the sum and sum of squares of each
// 64-column block they stored, as rounded, block-major; s comes from hdcm_row_sums_fwd, computed once per
// weight.  At its start a workgroup loads its 256 x 256 residual tile (16-byte runs, traded
// into the accumulator layout with v_permlane16_swap), reduces its 256 rows' partial sums to
// (mu_t, r_t) and starts the accumulators at res / r_t - mu_t * s_o; the epilogue then writes
// r_t * acc as 16-byte runs.  The residual's read overlaps the first operand tiles' loads and
// nothing is read after the K loop.  Measured in isolation at 32768 x 1024 x 1152: 86-90 us
// against 103-110 us for EPI_ROWLN (whose in-loop v_dot2 sums, reductions and 8-byte
// epilogue loads and stores make the difference).
//
// Workgroup order: workgroup b runs on XCD b % 8 (round-robin dispatch).  XCD x takes a
// contiguous run of tile indices, walked in bands of kGroup o-tiles (o fastest inside a
// band), so the ~32 workgroups resident on one XCD share a few W and X panels in its L2.
#include "hdcm_common.h"

using namespace hdcm;

namespace {

constexpr int kThreads = 512;
constexpr int kBO = 256, kBT = 256, kBK = 64;
constexpr int kChunks = kBK / 8;           // 16-byte chunks per tile row
constexpr int kGroup = 4;                  // o-tiles per band of the workgroup order
constexpr int kBufferFlags = 0x00020000;   // buffer resource word 3: raw 32-bit dwords
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

enum { EPI_BIAS = 0, EPI_ROWLN = 1, EPI_ROWSTATS = 2 };

__shared__ uint4 sW0[kBO * kChunks], sW1[kBO * kChunks], sX0[kBT * kChunks], sX1[kBT * kChunks];

// Tile (ot, tt) of this workgroup in the XCD-grouped order above.
__device__ __forceinline__ void tile_of(int n_otiles, int& ot, int& tt) {
  const int T = gridDim.x, b = blockIdx.x, x = b & 7, sl = b >> 3;
  int pre = 0;  // tiles taken by XCDs 0..x-1
  for (int y = 0; y < x; ++y) pre += (T - y + 7) >> 3;
  const int i = pre + sl;
  const int n_tt = T / n_otiles;
  const int band = i / (kGroup * n_tt), r = i - band * kGroup * n_tt;
  const int wb = min(kGroup, n_otiles - band * kGroup);
  tt = r / wb;
  ot = band * kGroup + (r - tt * wb);
}

template <int EPI, bool BIAS>
__global__ __launch_bounds__(kThreads, 1) void gemm_bt_kernel(
    const bf16_t* __restrict__ X, int64_t x_rs, const bf16_t* __restrict__ W, int64_t w_rs,
    const bf16_t* __restrict__ bias, const bf16_t* res, int64_t r_rs, bf16_t* out,
    int64_t o_rs, int M, int N, int K, int n_otiles, float eps, const float* __restrict__ wsum,
    const float* __restrict__ rstats, int nparts, int64_t stats_ps) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  int ot, tt;
  tile_of(n_otiles, ot, tt);
  const int o0 = ot * kBO, t0 = tt * kBT;
  const int nw = min(N - o0, kBO), nx = min(M - t0, kBT);
  const __amdgpu_buffer_rsrc_t wsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + (int64_t)o0 * w_rs), (short)0, (int)(((int64_t)(nw - 1) * w_rs + K) * 2), kBufferFlags);
  const __amdgpu_buffer_rsrc_t xsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(X + (int64_t)t0 * x_rs), (short)0, (int)(((int64_t)(nx - 1) * x_rs + K) * 2), kBufferFlags);

  // Loads: wave w fills rows 32 w + 8 i + lane / 8 (i < 4) of each operand; lane j lands in
  // LDS chunk j % 8 of its row, which holds global chunk (j % 8) ^ (row & 7).
  const int jr = lane >> 3, jc = (lane & 7) ^ jr;
  const int wvb = (int)(((int64_t)(w * 32 + jr) * w_rs + jc * 8) * 2);
  const int xvb = (int)(((int64_t)(w * 32 + jr) * x_rs + jc * 8) * 2);
  const int wst = (int)(8 * w_rs * 2), xst = (int)(8 * x_rs * 2);
  auto issue = [&](uint4* dw, uint4* dx, int k0) {
    // chunks past K take an offset past every buffer's end (2^31 + ...): they read zeros
    const bool kin = k0 + jc * 8 < K;
    const unsigned wv = kin ? (unsigned)(wvb + 2 * k0) : 0x80000000u;
    const unsigned xv = kin ? (unsigned)(xvb + 2 * k0) : 0x80000000u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wsrc, (lds_ptr_t)(dw + (w * 32 + 8 * i) * kChunks), 16,
                                               (int)(wv + (unsigned)(i * wst)), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xsrc, (lds_ptr_t)(dx + (w * 32 + 8 * i) * kChunks), 16,
                                               (int)(xv + (unsigned)(i * xst)), 0, 0, 0);
    }
  };

  const int wo = w & 1, wt = w >> 1;
  const int l16 = lane & 15, g = lane >> 4;
  // EPI_ROWSTATS lanes hold 8 consecutive columns for 16-byte runs: for the column tiles 2ip,
  // 2ip+1 of a row, lane group g takes columns 32 ip + gcol .. +7 (v_permlane16_swap trades
  // the 4+4 values of the MFMA layout between lanes g and g^1)
  const int gcol = 16 * (g & 1) + 8 * (g >> 1);
  f32x4_t acc[8][4];
  float rs[4] = {1.f, 1.f, 1.f, 1.f};
  if constexpr (EPI == EPI_ROWSTATS) {
    uint4 rraw[4][4];  // residual, 8 columns per (16-token tile j, column-tile pair ip)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = min(t0 + wt * 64 + j * 16 + l16, M - 1);
#pragma unroll
      for (int ip = 0; ip < 4; ++ip) {
        const int o = min(o0 + wo * 128 + ip * 32 + gcol, N - 8);
        rraw[j][ip] = *reinterpret_cast<const uint4*>(res + (int64_t)t * r_rs + o);
      }
    }
    float4 sv[8];  // s_o of the MFMA layout's columns o0 + 128 wo + 16 i + 4 g .. +3
#pragma unroll
    for (int i = 0; i < 8; ++i)
      sv[i] = *reinterpret_cast<const float4*>(wsum + min(o0 + wo * 128 + i * 16 + 4 * g, N - 4));
    issue(sW0, sX0, 0);
    // (mu, r) of the tile's rows.  Thread tid adds the partial sums of row t0 + tid % 256
    // with parts q = tid / 256, +2, +4, ... (part-major: 256 threads read 256 consecutive
    // pairs), 16 loads in flight at a time; the two halves meet in LDS.
    float2* mr = reinterpret_cast<float2*>(sW1);  // stage 1's buffer, loaded only after the loop's first barrier
    {
      constexpr int kBatch = 16;
      const int half = tid / kBT;
      const float2* ps = reinterpret_cast<const float2*>(rstats) + min(t0 + tid % kBT, M - 1);
      float s1 = 0.f, s2 = 0.f;
      for (int q0 = half; q0 < nparts; q0 += 2 * kBatch) {
        float2 v[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k)
          v[k] = q0 + 2 * k < nparts ? ps[(int64_t)(q0 + 2 * k) * stats_ps] : make_float2(0.f, 0.f);
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          s1 += v[k].x;
          s2 += v[k].y;
        }
      }
      mr[tid] = make_float2(s1, s2);  // [half][row]
    }
    __syncthreads();
    float mu[4];
    const float invK = 1.0f / (float)K;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = wt * 64 + j * 16 + l16;
      const float2 a = mr[row], b = mr[kBT + row];
      const float m = (a.x + b.x) * invK;
      mu[j] = m;
      rs[j] = rsqrtf(fmaxf((a.y + b.y) * invK - m * m, 0.f) + eps);
    }
    // acc = res / r - mu * s, so that r * (acc + c w^T) = res + r (c w^T - mu s)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float sd = 1.0f / rs[j];
#pragma unroll
      for (int ip = 0; ip < 4; ++ip) {
        const auto s0 = __builtin_amdgcn_permlane16_swap(rraw[j][ip].x, rraw[j][ip].z, false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(rraw[j][ip].y, rraw[j][ip].w, false, false);
        const uint32_t rw[2][2] = {{s0[0], s1[0]}, {s0[1], s1[1]}};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int i = 2 * ip + h;
          const float r4[4] = {__uint_as_float(rw[h][0] << 16), __uint_as_float(rw[h][0] & 0xffff0000u),
                               __uint_as_float(rw[h][1] << 16), __uint_as_float(rw[h][1] & 0xffff0000u)};
          const float s4[4] = {sv[i].x, sv[i].y, sv[i].z, sv[i].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][j][e] = fmaf(r4[e], sd, -mu[j] * s4[e]);
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  // EPI_ROWLN sums, taken in turns so each wave adds on a fraction of the K steps:
  //   ssum/ssq: sum c and sum c^2 of token l16 of the wave's j-th 16-token tile, on the K
  //   steps with kt % 2 == wo (the two waves sharing the tokens alternate);
  //   wsm: sum w of row l16 of the wave's i-th 16-row weight tile, on the K steps with
  //   kt % 4 == wt (the four waves sharing the rows take turns).
  float ssum[4] = {0.f, 0.f, 0.f, 0.f}, ssq[4] = {0.f, 0.f, 0.f, 0.f};
  float wsm[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const bf16x2_t ones = __builtin_bit_cast(bf16x2_t, 0x3f803f80u);

  auto compute = [&](const uint4* bw, const uint4* bx, int kt) {
    Frag<bf16_t> fa[2][8], fb[2][4];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int pcf = (kk * 4 + g) ^ (l16 & 7);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        fa[kk][i].v = __builtin_bit_cast(bf16x8_t, bw[(wo * 128 + i * 16 + l16) * kChunks + pcf]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        fb[kk][j].v = __builtin_bit_cast(bf16x8_t, bx[(wt * 64 + j * 16 + l16) * kChunks + pcf]);
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mma(fa[kk][i], fb[kk][j], acc[i][j]);
    // the first K half's 12 fragment reads, then the second half's 12 spread over the MFMAs
    __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
#pragma unroll
    for (int r = 0; r < 12; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 40, 0);
    if (EPI == EPI_ROWLN) {
      // after the MFMAs: these need every fragment of the step
      if ((kt & 1) == wo) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint4 u = __builtin_bit_cast(uint4, fb[kk][j].v);
            const unsigned d[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const bf16x2_t p = __builtin_bit_cast(bf16x2_t, d[e]);
              ssum[j] = __builtin_amdgcn_fdot2_f32_bf16(p, ones, ssum[j], false);
              ssq[j] = __builtin_amdgcn_fdot2_f32_bf16(p, p, ssq[j], false);
            }
          }
      }
      if ((kt & 3) == wt) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const uint4 u = __builtin_bit_cast(uint4, fa[kk][i].v);
            const unsigned d[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; ++e)
              wsm[i] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, d[e]), ones, wsm[i], false);
          }
      }
    }
  };

  const int nk = (K + kBK - 1) / kBK;
  if constexpr (EPI != EPI_ROWSTATS) issue(sW0, sX0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    const bool odd = kt & 1;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of tile kt are in LDS
    __syncthreads();                     // everyone's; and tile kt-1's buffer is free again
    if (kt + 1 < nk) issue(odd ? sW0 : sW1, odd ? sX0 : sX1, (kt + 1) * kBK);
    compute(odd ? sW1 : sW0, odd ? sX1 : sX0, kt);
  }

  if constexpr (EPI == EPI_ROWSTATS) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = t0 + wt * 64 + j * 16 + l16;
#pragma unroll
      for (int ip = 0; ip < 4; ++ip) {
        uint32_t w2[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const f32x4_t a = acc[2 * ip + h][j];
          w2[h][0] = pack_bf16x2(rs[j] * a[0], rs[j] * a[1]);
          w2[h][1] = pack_bf16x2(rs[j] * a[2], rs[j] * a[3]);
        }
        const auto s0 = __builtin_amdgcn_permlane16_swap(w2[0][0], w2[1][0], false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(w2[0][1], w2[1][1], false, false);
        const int o = o0 + wo * 128 + ip * 32 + gcol;
        if (t < M && o < N)
          *reinterpret_cast<uint4*>(out + (int64_t)t * o_rs + o) = make_uint4(s0[0], s1[0], s0[1], s1[1]);
      }
    }
    return;
  }
  uint2 rcur[8], rnext[8];
  auto load_res = [&](int j, uint2 (&r)[8]) {
    const int t = min(t0 + wt * 64 + j * 16 + l16, M - 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int o = min(o0 + wo * 128 + i * 16 + 4 * g, N - 4);
      r[i] = *reinterpret_cast<const uint2*>(res + (int64_t)t * r_rs + o);
    }
  };
  // the first residual rows are in flight while the statistics are reduced
  if (EPI == EPI_ROWLN) load_res(0, rcur);
  float mu[4] = {0.f, 0.f, 0.f, 0.f};  // rs (above) stays 1 for EPI_BIAS
  const float* wrow = nullptr;  // EPI_ROWLN: s of this tile's 256 weight rows, in LDS
  if (EPI == EPI_ROWLN) {
    // totals over the four lane groups, then over the waves sharing a row (LDS)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ssum[j] = quad_group_sum(ssum[j]);
      ssq[j] = quad_group_sum(ssq[j]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) wsm[i] = quad_group_sum(wsm[i]);
    __syncthreads();  // every wave is done with the tiles in LDS
    float* red = reinterpret_cast<float*>(sW0);  // [wo][256 tokens][2], then [wt][256 rows]
    float* wred = red + 2 * kBT * 2;
    if (g == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tk = wt * 64 + j * 16 + l16;
        red[(wo * kBT + tk) * 2] = ssum[j];
        red[(wo * kBT + tk) * 2 + 1] = ssq[j];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) wred[wt * kBO + wo * 128 + i * 16 + l16] = wsm[i];
    }
    __syncthreads();
    if (tid < kBO) wred[tid] += wred[kBO + tid] + wred[2 * kBO + tid] + wred[3 * kBO + tid];
    __syncthreads();
    wrow = wred;
    const float invK = 1.0f / (float)K;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int tk = wt * 64 + j * 16 + l16;
      const float s1 = red[tk * 2] + red[(kBT + tk) * 2];
      const float s2 = red[tk * 2 + 1] + red[(kBT + tk) * 2 + 1];
      mu[j] = s1 * invK;
      rs[j] = rsqrtf(fmaxf(s2 * invK - mu[j] * mu[j], 0.f) + eps);
    }
  }

  // epilogue: lane holds out[t][o .. o+3], t = t0 + 64 wt + 16 j + l16, o = o0 + 128 wo + 16 i + 4 g.
  // vmcnt counts stores as well as loads, so every load is issued ahead of the stores that
  // follow it: the column constants first, the residual rows one 16-token tile ahead.
  float cst[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int o = min(o0 + wo * 128 + i * 16 + 4 * g, N - 4);
    if (EPI == EPI_BIAS && BIAS) {
      const uint2 b = *reinterpret_cast<const uint2*>(bias + o);
      cst[i][0] = __uint_as_float(b.x << 16);
      cst[i][1] = __uint_as_float(b.x & 0xffff0000u);
      cst[i][2] = __uint_as_float(b.y << 16);
      cst[i][3] = __uint_as_float(b.y & 0xffff0000u);
    } else if (EPI == EPI_ROWLN) {
#pragma unroll
      for (int e = 0; e < 4; ++e) cst[i][e] = wrow[wo * 128 + i * 16 + 4 * g + e];
    } else {
      cst[i][0] = cst[i][1] = cst[i][2] = cst[i][3] = 0.f;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (EPI == EPI_ROWLN && j + 1 < 4) load_res(j + 1, rnext);
    const int t = t0 + wt * 64 + j * 16 + l16;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int o = o0 + wo * 128 + i * 16 + 4 * g;
      float v[4];
      if (EPI == EPI_BIAS) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][e] + cst[i][e];
      } else {
        const float rv[4] = {__uint_as_float(rcur[i].x << 16), __uint_as_float(rcur[i].x & 0xffff0000u),
                             __uint_as_float(rcur[i].y << 16), __uint_as_float(rcur[i].y & 0xffff0000u)};
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = rv[e] + rs[j] * (acc[i][j][e] - mu[j] * cst[i][e]);
      }
      if (t < M && o < N)
        *reinterpret_cast<uint2*>(out + (int64_t)t * o_rs + o) =
            make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    }
    if (EPI == EPI_ROWLN)
#pragma unroll
      for (int i = 0; i < 8; ++i) rcur[i] = rnext[i];
  }
}

// A workgroup's rows span at most 256 row strides of bytes, addressed with 32-bit offsets.
bool fits32(int64_t row_stride) { return row_stride <= ((int64_t)1 << 30) / (2 * kBO); }

int check_common(const void* x, int64_t x_rs, const void* w, int64_t w_rs, const void* out, int64_t o_rs, int64_t M,
                 int64_t N, int64_t K) {
  HDCM_CHECK_ARG(M >= 0 && N > 0 && K > 0, HDCM_EINVAL);
  HDCM_CHECK_ARG(w != nullptr && ((x && out) || M == 0), HDCM_EINVAL);
  HDCM_CHECK_ARG(w_rs >= K && (M == 0 || (x_rs >= K && o_rs >= N)), HDCM_EINVAL);
  HDCM_CHECK_ARG(K % 8 == 0 && N % 4 == 0 && x_rs % 8 == 0 && w_rs % 8 == 0 && o_rs % 4 == 0 &&
                     hdcm_aligned16(x) && hdcm_aligned16(w) && ((uintptr_t)out & 7u) == 0,
                 HDCM_EALIGN);
  HDCM_CHECK_ARG(M <= INT32_MAX && N <= INT32_MAX && fits32(x_rs) && fits32(w_rs), HDCM_EUNSUPPORTED);
  const int64_t tiles = ((N + kBO - 1) / kBO) * ((M + kBT - 1) / kBT);
  HDCM_CHECK_ARG(tiles <= INT32_MAX, HDCM_EUNSUPPORTED);
  return HDCM_OK;
}

}  // namespace

// skinny.hip: the row-LayerNorm fold on the decode-step kernels (M <= 16)
bool hdcm_skinny_rowln_ok(int64_t M, int64_t K);
int hdcm_skinny_rowln(const void* c, int64_t c_rs, const void* W, int64_t w_rs, const void* res, int64_t r_rs,
                      void* out, int64_t o_rs, int64_t M, int64_t N, int64_t K, float eps, hipStream_t s);

extern "C" int hdcm_gemm_fwd(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride,
                             const void* bias, void* out, int64_t out_row_stride, int64_t M, int64_t N, int64_t K,
                             int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  const int st = check_common(x, x_row_stride, w, w_row_stride, out, out_row_stride, M, N, K);
  if (st) return st;
  HDCM_CHECK_ARG(((uintptr_t)bias & 7u) == 0, HDCM_EALIGN);
  if (M == 0) return HDCM_OK;
  const int64_t n_ot = (N + kBO - 1) / kBO, n_tt = (M + kBT - 1) / kBT;
  auto kern = bias ? gemm_bt_kernel<EPI_BIAS, true> : gemm_bt_kernel<EPI_BIAS, false>;
  HDCM_LAUNCH(kern, dim3((unsigned)(n_ot * n_tt)), dim3(kThreads), 0, (hipStream_t)stream, (const bf16_t*)x,
                     x_row_stride, (const bf16_t*)w, w_row_stride, (const bf16_t*)bias, (const bf16_t*)nullptr,
                     (int64_t)0, (bf16_t*)out, out_row_stride, (int)M, (int)N, (int)K, (int)n_ot, 0.f,
                     (const float*)nullptr, (const float*)nullptr, 0, (int64_t)0);
  return hdcm_launch_status();
}

extern "C" int hdcm_rowln_gemm_fwd(const void* c, int64_t c_row_stride, const void* w, int64_t w_row_stride,
                                   const void* res, int64_t res_row_stride, void* out, int64_t out_row_stride, int64_t M,
                                   int64_t N, int64_t K, float eps, int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  const int st = check_common(c, c_row_stride, w, w_row_stride, out, out_row_stride, M, N, K);
  if (st) return st;
  HDCM_CHECK_ARG(res || M == 0, HDCM_EINVAL);
  HDCM_CHECK_ARG(M == 0 || res_row_stride >= N, HDCM_EINVAL);
  HDCM_CHECK_ARG(res_row_stride % 4 == 0 && ((uintptr_t)res & 7u) == 0, HDCM_EALIGN);
  if (M == 0) return HDCM_OK;
  if (hdcm_skinny_rowln_ok(M, K))  // a few rows (decode steps): the weight-streaming kernels
    return hdcm_skinny_rowln(c, c_row_stride, w, w_row_stride, res, res_row_stride, out, out_row_stride, M, N, K,
                             eps, (hipStream_t)stream);
  const int64_t n_ot = (N + kBO - 1) / kBO, n_tt = (M + kBT - 1) / kBT;
  HDCM_LAUNCH((gemm_bt_kernel<EPI_ROWLN, false>), dim3((unsigned)(n_ot * n_tt)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const bf16_t*)c, c_row_stride, (const bf16_t*)w, w_row_stride,
                     (const bf16_t*)nullptr, (const bf16_t*)res, res_row_stride, (bf16_t*)out, out_row_stride, (int)M,
                     (int)N, (int)K, (int)n_ot, eps, (const float*)nullptr, (const float*)nullptr, 0, (int64_t)0);
  return hdcm_launch_status();
}

namespace {

// s_o = sum_k W[o, k] in fp32, one wave per weight row.
__global__ __launch_bounds__(256) void row_sums_kernel(const bf16_t* __restrict__ W, int64_t w_rs, int N, int K,
                                                       float* __restrict__ sums) {
  const int o = blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (o >= N) return;
  const bf16_t* row = W + (int64_t)o * w_rs;
  float s = 0.f, q = 0.f;
  for (int k = 8 * lane; k < K; k += 8 * 64) {
    const uint4 v = *reinterpret_cast<const uint4*>(row + k);
    bf16_pair_sums(v.x, s, q);
    bf16_pair_sums(v.y, s, q);
    bf16_pair_sums(v.z, s, q);
    bf16_pair_sums(v.w, s, q);
  }
  s = wave_sum(s);
  if (lane == 0) sums[o] = s;
}

}  // namespace

extern "C" int hdcm_row_sums_fwd(const void* w, int64_t w_row_stride, int64_t N, int64_t K, float* sums,
                                 int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(N >= 0 && K > 0 && w_row_stride >= K && ((w && sums) || N == 0), HDCM_EINVAL);
  HDCM_CHECK_ARG(K % 8 == 0 && w_row_stride % 8 == 0 && hdcm_aligned16(w) && ((uintptr_t)sums & 3u) == 0,
                 HDCM_EALIGN);
  HDCM_CHECK_ARG(N <= ((int64_t)1 << 30), HDCM_EUNSUPPORTED);
  if (N == 0) return HDCM_OK;
  HDCM_LAUNCH(row_sums_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, (hipStream_t)stream, (const bf16_t*)w,
              w_row_stride, (int)N, (int)K, sums);
  return hdcm_launch_status();
}

extern "C" int hdcm_rowln_gemm_stats_fwd(const void* c, int64_t c_row_stride, const void* w, int64_t w_row_stride,
                                         const float* w_sums, const float* row_stats, int64_t stats_parts,
                                         int64_t stats_part_stride, const void* res, int64_t res_row_stride, void* out, int64_t out_row_stride,
                                         int64_t M, int64_t N, int64_t K, float eps, int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  const int st = check_common(c, c_row_stride, w, w_row_stride, out, out_row_stride, M, N, K);
  if (st) return st;
  HDCM_CHECK_ARG(M == 0 || (res && w_sums && row_stats), HDCM_EINVAL);
  HDCM_CHECK_ARG(M == 0 || res_row_stride >= N, HDCM_EINVAL);
  HDCM_CHECK_ARG(stats_parts >= 1 && stats_parts <= (1 << 20) && stats_part_stride >= M, HDCM_EINVAL);
  // 16-byte residual and output runs
  HDCM_CHECK_ARG(N % 8 == 0 && res_row_stride % 8 == 0 && out_row_stride % 8 == 0 && hdcm_aligned16(res) &&
                     hdcm_aligned16(out) && hdcm_aligned16(w_sums) && ((uintptr_t)row_stats & 7u) == 0,
                 HDCM_EALIGN);
  if (M == 0) return HDCM_OK;
  const int64_t n_ot = (N + kBO - 1) / kBO, n_tt = (M + kBT - 1) / kBT;
  HDCM_LAUNCH((gemm_bt_kernel<EPI_ROWSTATS, false>), dim3((unsigned)(n_ot * n_tt)), dim3(kThreads), 0,
              (hipStream_t)stream, (const bf16_t*)c, c_row_stride, (const bf16_t*)w, w_row_stride,
              (const bf16_t*)nullptr, (const bf16_t*)res, res_row_stride, (bf16_t*)out, out_row_stride, (int)M,
              (int)N, (int)K, (int)n_ot, eps, w_sums, row_stats, (int)stats_parts, stats_part_stride);
  return hdcm_launch_status();
}
