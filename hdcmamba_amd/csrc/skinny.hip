// Skinny bf16 GEMM for the single-token decode step on gfx950:
//   out[m, n] = sum_k A[m, k] W[n, k]  (+ bias[n])  (+ res[m, n]),   m < M <= 16
// with W an nn.Linear weight [N, K] (K contiguous).  It replaces the decode step's
// projections (in_proj with its bias, out_proj with the residual add; hdcmamba/model.py:313,
// 325,340,383 run them as nn.Linear).  The tied LM head (train_fineweb.py:55,94) takes it too
// but the model keeps the head on the library GEMM, which streams its 206 MB faster.
//
// At M = 16 every weight is read once per step and used for 16 rows only, so the GEMM is
// bound by streaming W from HBM.  Two kernels, both with one workgroup per 16-column tile
// of the output and every load of a wave issued before its first v_mfma_f32_16x16x32_bf16:
//   skinny_gemm_kernel: four waves split K four ways; each lane loads its MFMA fragments
//     straight from W (16 rows x 64 contiguous bytes per instruction).
//   skinny_lds_kernel (N >= 2048, where it is faster): eight waves split K eight ways; a
//     wave reads its K range of the 16 rows row-major (a few hundred contiguous bytes of a
//     row per instruction) into a private LDS slab and takes the fragments from there.
// A (the 16 activation rows, a few tens of KB) is read from L2.  The partial 16x16 tiles are
// summed through LDS and the epilogue adds bias and residual (loaded at the start, so no load
// waits behind the MFMAs) in fp32 and rounds once to bf16.
#include <atomic>

#include "hdcm_common.h"

using namespace hdcm;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxSteps = 24;  // K=32 steps per wave: K <= 4 * 24 * 32 = 3072

// Row LayerNorm folded in (LN): out = res + r_m (acc - mu_m s_n), LN(c) W^T written through
// the sums of the operands the MFMAs read: lane (l16, g) adds its A fragment's sum c and sum
// c^2 (row m = l16) and its B fragment's sum w (column n = l16) with v_dot2_f32_bf16; the
// four lane groups are added on lane moves and the waves' K ranges in LDS.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void ln_sums(const Frag<bf16_t>& a, const Frag<bf16_t>& b, float& c1, float& c2,
                                        float& w1) {
  const bf16x2_t ones = __builtin_bit_cast(bf16x2_t, 0x3f803f80u);
  const uint4 ua = __builtin_bit_cast(uint4, a.v), ub = __builtin_bit_cast(uint4, b.v);
  const unsigned da[4] = {ua.x, ua.y, ua.z, ua.w}, db[4] = {ub.x, ub.y, ub.z, ub.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const bf16x2_t p = __builtin_bit_cast(bf16x2_t, da[e]);
    c1 = __builtin_amdgcn_fdot2_f32_bf16(p, ones, c1, false);
    c2 = __builtin_amdgcn_fdot2_f32_bf16(p, p, c2, false);
    w1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, db[e]), ones, w1, false);
  }
}
__device__ __forceinline__ void ln_store(float (&st)[16][3], int l16, int g, float c1, float c2, float w1) {
  c1 = quad_group_sum(c1);
  c2 = quad_group_sum(c2);
  w1 = quad_group_sum(w1);
  if (g == 0) {
    st[l16][0] = c1;
    st[l16][1] = c2;
    st[l16][2] = w1;
  }
}
template <int NW>
__device__ __forceinline__ float ln_apply(const float (&st)[NW][16][3], int m, int nn, int K, float eps, float acc) {
  float s1 = 0.f, s2 = 0.f, sw = 0.f;
#pragma unroll
  for (int k = 0; k < NW; ++k) {
    s1 += st[k][m][0];
    s2 += st[k][m][1];
    sw += st[k][nn][2];
  }
  const float mu = s1 / (float)K;
  const float r = rsqrtf(fmaxf(s2 / (float)K - mu * mu, 0.f) + eps);
  return r * (acc - mu * sw);
}

template <int STEPS, bool BIAS, bool RES, bool LN = false>
__global__ __launch_bounds__(kThreads) void skinny_gemm_kernel(
    const bf16_t* __restrict__ A, int64_t a_rs, const bf16_t* __restrict__ W, int64_t w_rs,
    const bf16_t* __restrict__ bias, const bf16_t* __restrict__ res, int64_t r_rs,
    bf16_t* __restrict__ out, int64_t o_rs, int M, int N, int K, float eps = 0.f) {
  __shared__ float part[kWaves][16][17];
  __shared__ float lnst[LN ? kWaves : 1][16][3];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int l16 = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int nsteps = K / 32;
  // contiguous K ranges per wave: the first (nsteps % 4) waves take one step more
  const int base = nsteps / kWaves, extra = nsteps % kWaves;
  const int my = base + (w < extra ? 1 : 0);
  const int s0 = w * base + (w < extra ? w : extra);

  // A fragments: lane (m = l16, g) holds A[m][32 s + 8 g .. +8]; rows past M read row 0.
  // B fragments: lane (n = l16, g) holds W[n0 + n][32 s + 8 g .. +8]; rows past N read row
  // N-1 (their outputs are not stored).  Every load of the wave is issued before the first
  // MFMA (A first: it is L2-resident and returns ahead of W), so the wave waits for one
  // memory round trip instead of one per K step.
  // the epilogue's bias and residual values, loaded now so the epilogue waits for nothing
  // (branch-free at clamped addresses, converted in the epilogue: see skinny_lds_kernel)
  const int en = min(n0 + l16, N - 1);
  bf16_t eb{}, er[4] = {};
  if constexpr (BIAS) eb = bias[en];
  if constexpr (RES) {
#pragma unroll
    for (int r = 0; r < 4; ++r) er[r] = res[(int64_t)min(4 * g + r, M - 1) * r_rs + en];
  }
  const int am = l16 < M ? l16 : 0;
  const bf16_t* ap = A + (int64_t)am * a_rs + 8 * g;
  const int wn = min(n0 + l16, N - 1);
  const bf16_t* wp = W + (int64_t)wn * w_rs + 8 * g;
  Frag<bf16_t> fa[STEPS], bw[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s)
    if (s < my) fa[s].v = *reinterpret_cast<const bf16x8_t*>(ap + 32 * (s0 + s));
#pragma unroll
  for (int s = 0; s < STEPS; ++s)
    if (s < my) bw[s].v = *reinterpret_cast<const bf16x8_t*>(wp + 32 * (s0 + s));
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < STEPS; ++s)
    if (s < my) acc = mma(fa[s], bw[s], acc);
  if constexpr (LN) {
    float c1 = 0.f, c2 = 0.f, w1 = 0.f;
#pragma unroll
    for (int s = 0; s < STEPS; ++s)
      if (s < my) ln_sums(fa[s], bw[s], c1, c2, w1);
    ln_store(lnst[w], l16, g, c1, c2, w1);
  }
  // D layout: lane holds D[4 g + r][l16]
#pragma unroll
  for (int r = 0; r < 4; ++r) part[w][4 * g + r][l16] = acc[r];
  __syncthreads();
  if (w == 0) {
    const int n = n0 + l16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * g + r;
      float v = part[0][m][l16] + part[1][m][l16] + part[2][m][l16] + part[3][m][l16];
      float pre = 0.f;
      if constexpr (BIAS) pre += bf2f(eb);
      if constexpr (RES) pre += bf2f(er[r]);
      if (m < M && n < N) {
        if constexpr (LN) v = ln_apply<kWaves>(lnst, m, l16, K, eps, v);
        out[(int64_t)m * o_rs + n] = f2bf(v + pre);
      }
    }
  }
}

// Wide outputs (N >= kWideN): a workgroup of 8 waves per 16 output columns, each wave owning a
// contiguous K range of the 16 weight rows.  A wave reads its range row by row (lane i of
// load instruction j takes 16-byte piece 64*j + i of the range, row-major), so one instruction
// covers about two rows with a few hundred contiguous bytes each instead of 16 rows x 64
// bytes, and stages it in a private LDS slab, from which the B fragments are read.  Every
// lane issues the same number of loads (pieces past the wave's range re-read one inside the
// row and are never used), so all loads are in flight before the first wait.
// NCOL (16 or 8) output columns per workgroup: with 8, a workgroup streams 8 weight rows and
// the MFMA's other 8 columns repeat them (their outputs are not stored), which doubles the
// workgroups of a narrow output (the d_model 2048 out_proj: 256 instead of 128, every CU
// streaming) at the cost of reading the activation rows twice as often from L2.
constexpr int kLdsWaves = 8;
constexpr int kLdsThreads = kLdsWaves * kWave;
constexpr int kWideN = 2048;
// outputs of the LDS kernel up to this width use 8-column workgroups (HDCM_OPT_SKINNY_COLS8_MAX_N)
inline bool cols8(int N) { return N <= hdcm_option_value(HDCM_OPT_SKINNY_COLS8_MAX_N); }

// Second tiles (without LN): a launch of more column tiles than fit on the GPU at once would
// run its last tiles as a second round of workgroups, each paying the full load latency again.
// Instead the grid is one round and workgroup i < second_tiles also computes tile gridDim.x + i: its
// waves load that tile's B fragments straight from W into registers (16 rows x 64 bytes per
// instruction) together with the slab loads, reuse the A fragments, and sum the partial tiles
// through their own slab regions (`second_tiles` of them).  Same K split and summation order, so the values are those
// of a workgroup of its own.
template <int STEPS, bool BIAS, bool RES, bool LN = false, int NCOL = 16>
__global__ __launch_bounds__(kLdsThreads) void skinny_lds_kernel(
    const bf16_t* __restrict__ A, int64_t a_rs, const bf16_t* __restrict__ W, int64_t w_rs,
    const bf16_t* __restrict__ bias, const bf16_t* __restrict__ res, int64_t r_rs,
    bf16_t* __restrict__ out, int64_t o_rs, int M, int N, int K, float eps, int second_tiles) {
  static_assert(NCOL == 16 || NCOL == 8, "columns per workgroup");
  constexpr int PITCH = STEPS * 32 + 8;  // slab row pitch (elements): +16 bytes staggers the banks
  constexpr int NLD = (NCOL * 4 * STEPS + kWave - 1) / kWave;  // 16-byte weight loads per lane
  __shared__ __attribute__((aligned(16))) bf16_t slab[kLdsWaves][NCOL * PITCH];
  __shared__ float part[kLdsWaves][16][17];
  __shared__ float lnst[LN ? kLdsWaves : 1][16][3];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int l16 = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * NCOL;
  const int nsteps = K / 32;
  const int base = nsteps / kLdsWaves, extra = nsteps % kLdsWaves;
  const int my = base + (w < extra ? 1 : 0);
  const int s0 = w * base + (w < extra ? w : extra);
  // the K step a slot s < STEPS of this wave reads: its own, or (past its range) one inside the row
  auto step_of = [&](int s) { return min(s0 + max(min(s, my - 1), 0), nsteps - 1); };

  // second tile (see above): uniform per workgroup
  const bool two = !LN && (int)blockIdx.x < second_tiles;
  const int n1 = ((int)gridDim.x + (int)blockIdx.x) * NCOL;
  // the epilogue's bias and residual values, loaded now so the epilogue waits for nothing
  // (thread tid < 16*NCOL: row tid / NCOL, column tid % NCOL)
  // (branch-free, at clamped addresses, and converted only in the epilogue: a load whose
  // value is converted inside a branch is waited for there, ahead of the weight loads)
  const int em = min(tid / NCOL, M - 1), en0 = min(n0 + tid % NCOL, N - 1), en1 = min(n1 + tid % NCOL, N - 1);
  bf16_t eb0{}, eb1{}, er0{}, er1{};
  if constexpr (BIAS) eb0 = bias[en0], eb1 = bias[en1];
  if constexpr (RES) er0 = res[(int64_t)em * r_rs + en0], er1 = res[(int64_t)em * r_rs + en1];
  // the second tile's B fragments, issued first (the slab and A loads after them are then
  // waited for with the same counts on both paths): lane (l16, g) takes row n1 + l16 % NCOL
  Frag<bf16_t> b1[LN ? 1 : STEPS];
  if constexpr (!LN) {
    if (two) {
      const bf16_t* w1p = W + (int64_t)min(n1 + l16 % NCOL, N - 1) * w_rs + 8 * g;
#pragma unroll
      for (int s = 0; s < STEPS; ++s) b1[s].v = *reinterpret_cast<const bf16x8_t*>(w1p + 32 * step_of(s));
    }
  }
  // piece idx of the wave's NCOL rows x STEPS steps x 4 sixteen-byte quarters; indices past
  // them (NCOL*STEPS not a multiple of 16) re-read the last piece and are not staged
  auto piece = [&](int i, int& r, int& st, int& q) {
    const int idx = min(kWave * i + lane, NCOL * 4 * STEPS - 1);
    r = idx / (4 * STEPS), st = (idx / 4) % STEPS, q = idx % 4;
  };
  uint4 raw[NLD];
#pragma unroll
  for (int i = 0; i < NLD; ++i) {
    int r, st, q;
    piece(i, r, st, q);
    const int n = min(n0 + r, N - 1);  // rows past N re-read row N-1 (outputs not stored)
    raw[i] = *reinterpret_cast<const uint4*>(W + (int64_t)n * w_rs + 32 * step_of(st) + 8 * q);
  }
  const int am = l16 < M ? l16 : 0;  // rows past M read row 0 (outputs not stored)
  Frag<bf16_t> fa[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s)
    fa[s].v = *reinterpret_cast<const bf16x8_t*>(A + (int64_t)am * a_rs + 32 * step_of(s) + 8 * g);
  bf16_t* sl = slab[w];
#pragma unroll
  for (int i = 0; i < NLD; ++i) {
    int r, st, q;
    piece(i, r, st, q);
    if (kWave * i + lane < NCOL * 4 * STEPS) *reinterpret_cast<uint4*>(sl + r * PITCH + 32 * st + 8 * q) = raw[i];
  }
  __syncthreads();
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  float c1 = 0.f, c2 = 0.f, w1 = 0.f;
  const int br = l16 % NCOL;  // B column l16 reads slab row l16 mod NCOL
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    if (s < my) {
      Frag<bf16_t> b;
      b.v = *reinterpret_cast<const bf16x8_t*>(sl + br * PITCH + 32 * s + 8 * g);
      acc = mma(fa[s], b, acc);
      if constexpr (LN) ln_sums(fa[s], b, c1, c2, w1);
    }
  }
  if constexpr (LN) ln_store(lnst[w], l16, g, c1, c2, w1);
  // D layout: lane holds D[4 g + r][l16]
#pragma unroll
  for (int r = 0; r < 4; ++r) part[w][4 * g + r][l16] = acc[r];
  // the second tile's partial goes to the start of this wave's own slab, whose reads are done
  // (a wave's LDS accesses complete in order; the empty asm keeps the compiler from moving the
  // float stores above the bf16 reads of the same bytes)
  static_assert(NCOL * PITCH * sizeof(bf16_t) >= 16 * 17 * sizeof(float), "slab holds a partial tile");
  float* part1 = reinterpret_cast<float*>(sl);
  if constexpr (!LN) {
    if (two) {
      asm volatile("" ::: "memory");
      f32x4_t acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < STEPS; ++s)
        if (s < my) acc1 = mma(fa[s], b1[s], acc1);
#pragma unroll
      for (int r = 0; r < 4; ++r) part1[(4 * g + r) * 17 + l16] = acc1[r];
    }
  }
  __syncthreads();
  if (tid < 16 * NCOL) {
    const int m = tid / NCOL, nn = tid % NCOL, n = n0 + nn;
    float v = 0.f;
#pragma unroll
    for (int k = 0; k < kLdsWaves; ++k) v += part[k][m][nn];
    float pre = 0.f, pre1 = 0.f;
    if constexpr (BIAS) pre += bf2f(eb0), pre1 += bf2f(eb1);
    if constexpr (RES) pre += bf2f(er0), pre1 += bf2f(er1);
    if (m < M && n < N) {
      if constexpr (LN) v = ln_apply<kLdsWaves>(lnst, m, nn, K, eps, v);
      out[(int64_t)m * o_rs + n] = f2bf(v + pre);
    }
    if (two) {
      float v1 = 0.f;
#pragma unroll
      for (int k = 0; k < kLdsWaves; ++k) v1 += reinterpret_cast<const float*>(slab[k])[m * 17 + nn];
      if (m < M && n1 + nn < N) out[(int64_t)m * o_rs + n1 + nn] = f2bf(v1 + pre1);
    }
  }
}

// ------------------------------------------------------------ fused front of the decode step
// The step's LayerNorm + causal conv of the new token (norm_conv_step, hdcmamba/model.py:22-72
// one row at a time) and the in_proj skinny GEMM over its output (model.py:313,340) in one
// launch.  Apart, the GEMM's 35 MB weight stream (d_model 2048) could only start once the
// conv kernel had ended; here it is in flight while the conv rows are computed:
//   workgroups 0..M-1 (dispatched first) each compute one row u_m exactly as
//     norm_conv_step_kernel does (waves 0-3, one 16-byte group per thread, the same sums in
//     the same order), shift that row's history, store u_m with agent-scope (sc1) stores,
//     wait for them and publish flag m = the call's tag;
//   workgroups M.. are skinny_lds_kernel<STEPS, bias, -, -, 16> workgroups (second tiles
//     included): they issue their weight loads first, then wave 0 polls the M flags
//     (agent-scope loads; its first poll returns once its own weight loads are in), and only
//     after that barrier are the A fragments read from u.
// No workgroup reads u before its flag is seen in this launch, and a launch begins with the
// caches of the previous launches' data invalidated, so the A loads cannot hit a stale line.
// The call's tag lives in the workspace (as in the scan): every workgroup reads it and counts
// its arrival once it has; the last to arrive stores the next tag when it ends, so flags of
// earlier calls never match.  A wait that exceeds `spin_rounds` polls (HDCM_OPT_STEP_SPIN_ROUNDS)
// counts a timeout and goes on, so every wave exits after a bounded wait; the producers are the
// lowest workgroup indices and wait for nothing, so a timeout does not occur unless the GPU is
// shared with work that keeps them from being dispatched.
// Workspace lines (128 bytes each; a line that takes a grid's worth of atomics serialises every
// access to it, measured at ~40 us for 512 arrivals next to the tag and the flags, so each
// kind of access has lines of its own): the tag; the timeout count; eight copies of the M row
// flags, workgroup b polling copy b % 8; eight arrival counters, workgroup b counting in
// counter b % 8; and a ninth counter of the completed eight.
constexpr int kStepMaxRows = 16;
constexpr int kStepLine = 32;  // u32 words per 128-byte line
constexpr int kStepTag = 0, kStepTimeouts = kStepLine, kStepFlags = 2 * kStepLine;
constexpr int kStepGroups = 8;
constexpr int kStepCounters = kStepFlags + kStepGroups * kStepLine;
constexpr int kStepTotal = kStepCounters + kStepGroups * kStepLine;
constexpr size_t kStepWsBytes = (size_t)(kStepTotal + kStepLine) * sizeof(unsigned);
constexpr int kCachePolicySC1 = 16;  // buffer store cache policy: agent-scope coherent (sc1)
constexpr int kBufferFlags = 0x00020000;   // buffer resource word 3: raw 32-bit dwords
typedef unsigned v4u32_t __attribute__((ext_vector_type(4)));

// Arrival of this workgroup in counter blockIdx % 8, issued once the call's tag has been read
// (the asm needs its value): one lane's atomic, whose result is needed only at the end.
__device__ __forceinline__ unsigned step_arrive(unsigned* ws, unsigned tag) {
  unsigned arrived = 0;
  if (threadIdx.x == 0) {
    unsigned zero;
    __asm__ volatile("v_mov_b32 %0, 0" : "=v"(zero) : "v"(tag));
    arrived = __hip_atomic_fetch_add(ws + kStepCounters + kStepLine * (blockIdx.x % kStepGroups) + zero, 1u,
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return arrived;
}
// The workgroup that completes its counter counts it in the ninth; the one that completes that
// (every workgroup has read the tag) clears the counters and stores the next call's tag.
__device__ __forceinline__ void step_finish(unsigned* ws, unsigned tag, unsigned arrived) {
  if (threadIdx.x != 0) return;
  const unsigned G = gridDim.x, x = blockIdx.x % kStepGroups;
  if (arrived != (G - x + kStepGroups - 1) / kStepGroups - 1) return;
  const unsigned groups = G < (unsigned)kStepGroups ? G : (unsigned)kStepGroups;
  if (__hip_atomic_fetch_add(ws + kStepTotal, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != groups - 1) return;
  for (int y = 0; y < kStepGroups; ++y)
    __hip_atomic_store(ws + kStepCounters + kStepLine * y, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(ws + kStepTotal, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(ws + kStepTag, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int STEPS>
__global__ __launch_bounds__(kLdsThreads) void nc_in_step_kernel(
    const bf16_t* __restrict__ x, int64_t x_rs, const bf16_t* __restrict__ ln_w, const bf16_t* __restrict__ ln_b,
    const bf16_t* __restrict__ conv_w, const bf16_t* __restrict__ conv_b, bf16_t* __restrict__ hist, float eps,
    bf16_t* u, int64_t u_rs, const bf16_t* __restrict__ W, int64_t w_rs, const bf16_t* __restrict__ bias,
    bf16_t* __restrict__ out, int64_t o_rs, int M, int N, int K, int second_tiles, unsigned* ws,
    int spin_rounds) {
  constexpr int NCOL = 16;
  constexpr int PITCH = STEPS * 32 + 8;
  constexpr int NLD = (NCOL * 4 * STEPS + kWave - 1) / kWave;
  constexpr int kConvThreads = 256;  // the conv rows' threads: waves 0-3, one 16-byte group each
  __shared__ __attribute__((aligned(16))) bf16_t slab[kLdsWaves][NCOL * PITCH];
  __shared__ float part[kLdsWaves][16][17];
  __shared__ float red[kConvThreads / kWave * 8];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  // the call's tag, read behind each path's first loads (not waited for ahead of them)
  auto read_tag = [&]() { return __hip_atomic_load(ws + kStepTag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u; };

  if ((int)blockIdx.x < M) {
    // ---- conv row m (norm_conv_step_kernel<bf16_t, 1>'s arithmetic)
    const int m = blockIdx.x;
    const int G = K / 8;
    const bool act = tid < G;  // G <= 256: waves 4-7 only join the barriers
    const int gi = act ? tid : 0;
    const bf16_t* rows[4] = {hist + ((int64_t)m * 3 + 0) * K, hist + ((int64_t)m * 3 + 1) * K,
                             hist + ((int64_t)m * 3 + 2) * K, x + (int64_t)m * x_rs};
    uint4 raw[4], prm[7];
#pragma unroll
    for (int k = 0; k < 4; ++k) raw[k] = ldg16(rows[k] + gi * 8);
    prm[0] = ldg16(ln_w + gi * 8);
    prm[1] = ldg16(ln_b + gi * 8);
    prm[2] = ldg16(conv_b + gi * 8);
#pragma unroll
    for (int k = 0; k < 4; ++k) prm[3 + k] = ldg16(conv_w + (int64_t)gi * 32 + k * 8);
    const unsigned tag = read_tag();
    float r[4][8], st[8];
#pragma unroll
    for (int n = 0; n < 8; ++n) st[n] = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      unpack16<bf16_t>(raw[k], r[k]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = act ? r[k][e] : 0.f;
        st[2 * k] += v;
        st[2 * k + 1] += v * v;
      }
    }
    // workgroup sums over waves 0-3 (block_sum<8> of the conv kernel)
#pragma unroll
    for (int n = 0; n < 8; ++n) st[n] = wave_sum(st[n]);
    if (lane == 0 && w < kConvThreads / kWave) {
#pragma unroll
      for (int n = 0; n < 8; ++n) red[w * 8 + n] = st[n];
    }
    __syncthreads();
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      float s = 0.f;
#pragma unroll
      for (int k = 0; k < kConvThreads / kWave; ++k) s += red[k * 8 + n];
      st[n] = s;
    }
    float mean[4], rstd[4];
    const float invD = 1.0f / (float)K;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      mean[k] = st[2 * k] * invD;
      const float var = fmaxf(st[2 * k + 1] * invD - mean[k] * mean[k], 0.f);
      rstd[k] = rsqrtf(var + eps);
    }
    if (act) {
      float wv[8], bb[8], cb[8], cw[32], o[8];
      unpack16<bf16_t>(prm[0], wv);
      unpack16<bf16_t>(prm[1], bb);
      unpack16<bf16_t>(prm[2], cb);
#pragma unroll
      for (int k = 0; k < 4; ++k) unpack16<bf16_t>(prm[3 + k], cw + k * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float acc = cb[e];
#pragma unroll
        for (int k = 0; k < 4; ++k) acc += ((r[k][e] - mean[k]) * rstd[k] * wv[e] + bb[e]) * cw[4 * e + k];
        o[e] = acc;
      }
      const __amdgpu_buffer_rsrc_t usrc =
          __builtin_amdgcn_make_buffer_rsrc((void*)(u + (int64_t)m * u_rs), (short)0, K * 2, kBufferFlags);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32_t, pack16<bf16_t>(o)), usrc, tid * 16, 0,
                                             kCachePolicySC1);
#pragma unroll
      for (int k = 0; k < 3; ++k) *reinterpret_cast<uint4*>(hist + ((int64_t)m * 3 + k) * K + tid * 8) = raw[k + 1];
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's u stores have completed at agent scope
    __syncthreads();
    if (tid < kStepGroups)  // the flag, in each of the eight copies
      __hip_atomic_store(ws + kStepFlags + kStepLine * tid + m, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the arrival only now: a returning atomic issued before the u stores would have been
    // waited for with them
    step_finish(ws, tag, step_arrive(ws, tag));
  } else {
    // ---- in_proj column tiles (skinny_lds_kernel<STEPS, bias, false, false, 16>)
    const int j = (int)blockIdx.x - M, ng = (int)gridDim.x - M;
    const int n0 = j * NCOL;
    const int nsteps = K / 32;
    const int base = nsteps / kLdsWaves, extra = nsteps % kLdsWaves;
    const int my = base + (w < extra ? 1 : 0);
    const int s0 = w * base + (w < extra ? w : extra);
    auto step_of = [&](int s) { return min(s0 + max(min(s, my - 1), 0), nsteps - 1); };
    const bool two = j < second_tiles;
    const int n1 = (ng + j) * NCOL;
    // bias values for the epilogue (branch-free, converted there; see skinny_lds_kernel)
    const bf16_t* bp = bias != nullptr ? bias : W;
    const bf16_t eb0 = bp[min(n0 + tid % NCOL, N - 1)], eb1 = bp[min(n1 + tid % NCOL, N - 1)];
    Frag<bf16_t> b1[STEPS];
    if (two) {
      const bf16_t* w1p = W + (int64_t)min(n1 + (lane & 15), N - 1) * w_rs + 8 * (lane >> 4);
#pragma unroll
      for (int s = 0; s < STEPS; ++s) b1[s].v = *reinterpret_cast<const bf16x8_t*>(w1p + 32 * step_of(s));
    }
    auto piece = [&](int i, int& r, int& st, int& q) {
      const int idx = min(kWave * i + lane, NCOL * 4 * STEPS - 1);
      r = idx / (4 * STEPS), st = (idx / 4) % STEPS, q = idx % 4;
    };
    v4u32_t raw[NLD];  // a native vector type: plain loads and stores, no copies through memory
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      int r, st, q;
      piece(i, r, st, q);
      const int n = min(n0 + r, N - 1);
      raw[i] = *reinterpret_cast<const v4u32_t*>(W + (int64_t)n * w_rs + 32 * step_of(st) + 8 * q);
    }
    const unsigned tag = read_tag();
    // wait for the M conv rows (this workgroup's copy of the flags)
    if (w == 0) {
      const unsigned* flags = ws + kStepFlags + kStepLine * (blockIdx.x % kStepGroups);
      int polls = 0;
      while (true) {
        const bool ok = lane >= M || __hip_atomic_load(flags + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == tag;
        if (__all(ok)) break;
        if (++polls > spin_rounds) {
          if (lane == 0) __hip_atomic_fetch_add(ws + kStepTimeouts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    __syncthreads();
    const unsigned arrived = step_arrive(ws, tag);
    // The A loads take an offset from an asm placed after the wait, so they cannot be issued
    // ahead of it (a memory clobber would also pin the weight registers to memory; an asm on
    // the pointer itself would turn them into flat loads).
    int64_t uoff = 0;
    __asm__ volatile("" : "+s"(uoff));
    const bf16_t* ua = u + uoff;
    const int l16 = lane & 15, g = lane >> 4;
    const int am = l16 < M ? l16 : 0;
    Frag<bf16_t> fa[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s)
      fa[s].v = *reinterpret_cast<const bf16x8_t*>(ua + (int64_t)am * u_rs + 32 * step_of(s) + 8 * g);
    bf16_t* sl = slab[w];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      int r, st, q;
      piece(i, r, st, q);
      if (kWave * i + lane < NCOL * 4 * STEPS) *reinterpret_cast<v4u32_t*>(sl + r * PITCH + 32 * st + 8 * q) = raw[i];
    }
    __syncthreads();
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      if (s < my) {
        Frag<bf16_t> b;
        b.v = *reinterpret_cast<const bf16x8_t*>(sl + l16 * PITCH + 32 * s + 8 * g);
        acc = mma(fa[s], b, acc);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) part[w][4 * g + r][l16] = acc[r];
    float* part1 = reinterpret_cast<float*>(sl);
    if (two) {
      asm volatile("" ::: "memory");
      f32x4_t acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < STEPS; ++s)
        if (s < my) acc1 = mma(fa[s], b1[s], acc1);
#pragma unroll
      for (int r = 0; r < 4; ++r) part1[(4 * g + r) * 17 + l16] = acc1[r];
    }
    __syncthreads();
    if (tid < 16 * NCOL) {
      const int mm = tid / NCOL, nn = tid % NCOL, n = n0 + nn;
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < kLdsWaves; ++k) v += part[k][mm][nn];
      const float pre = bias != nullptr ? 0.f + bf2f(eb0) : 0.f, pre1 = bias != nullptr ? 0.f + bf2f(eb1) : 0.f;
      if (mm < M && n < N) out[(int64_t)mm * o_rs + n] = f2bf(v + pre);
      if (two) {
        float v1 = 0.f;
#pragma unroll
        for (int k = 0; k < kLdsWaves; ++k) v1 += reinterpret_cast<const float*>(slab[k])[mm * 17 + nn];
        if (mm < M && n1 + nn < N) out[(int64_t)mm * o_rs + n1 + nn] = f2bf(v1 + pre1);
      }
    }
    step_finish(ws, tag, arrived);
  }
}

// Workgroups of `kernel` (kLdsThreads threads) resident at once on the current device
// (occupancy per CU x CUs), found once per device and kernel; 0 if the runtime cannot tell.
template <typename Kernel>
int resident_wgs(Kernel kernel, std::atomic<int> (&cache)[16]) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kLdsThreads, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      per_cu = cus = 0;
    v = per_cu > 0 && cus > 0 ? per_cu * cus : -1;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v > 0 ? v : 0;
}

// Workgroups of skinny_lds_kernel<STEPS, BIAS, RES, false, NCOL> resident at once.
template <int STEPS, bool BIAS, bool RES, int NCOL>
int lds_resident() {
  static std::atomic<int> cache[16];
  return resident_wgs(skinny_lds_kernel<STEPS, BIAS, RES, false, NCOL>, cache);
}

template <int STEPS>
int launch_nc_in(const bf16_t* x, int64_t x_rs, const bf16_t* ln_w, const bf16_t* ln_b, const bf16_t* conv_w,
                 const bf16_t* conv_b, bf16_t* hist, float eps, bf16_t* u, int64_t u_rs, const bf16_t* W,
                 int64_t w_rs, const bf16_t* bias, bf16_t* out, int64_t o_rs, int M, int N, int K, unsigned* hdr,
                 hipStream_t s) {
  static std::atomic<int> cache[16];
  const int tiles = (N + 15) / 16;
  int gemm = tiles, extra = 0;
  if (hdcm_option_value(HDCM_OPT_SKINNY_FOLD_TAIL)) {
    const int res_wgs = resident_wgs(nc_in_step_kernel<STEPS>, cache) - M;
    if (res_wgs > 0 && tiles > res_wgs && tiles <= 2 * res_wgs) {
      gemm = res_wgs;
      extra = tiles - res_wgs;
    }
  }
  HDCM_LAUNCH((nc_in_step_kernel<STEPS>), dim3((unsigned)(M + gemm)), dim3(kLdsThreads), 0, s, x, x_rs, ln_w, ln_b,
              conv_w, conv_b, hist, eps, u, u_rs, W, w_rs, bias, out, o_rs, M, N, K, extra, hdr,
              hdcm_option_value(HDCM_OPT_STEP_SPIN_ROUNDS));
  return hdcm_launch_status();
}

// One round of workgroups with second tiles when the tiles exceed one round by at most a
// round (HDCM_OPT_SKINNY_FOLD_TAIL); otherwise a workgroup per tile.
template <int STEPS, bool BIAS, bool RES, int NCOL>
void launch_lds_one(const bf16_t* a, int64_t a_rs, const bf16_t* wt, int64_t w_rs, const bf16_t* bs,
                    const bf16_t* rs, int64_t r_rs, bf16_t* o, int64_t o_rs, int M, int N, int K, hipStream_t s) {
  const int tiles = (N + NCOL - 1) / NCOL;
  int grid = tiles, extra = 0;
  if (hdcm_option_value(HDCM_OPT_SKINNY_FOLD_TAIL)) {
    const int res_wgs = lds_resident<STEPS, BIAS, RES, NCOL>();
    if (res_wgs > 0 && tiles > res_wgs && tiles <= 2 * res_wgs) {
      grid = res_wgs;
      extra = tiles - res_wgs;
    }
  }
  HDCM_LAUNCH((skinny_lds_kernel<STEPS, BIAS, RES, false, NCOL>), dim3((unsigned)grid), dim3(kLdsThreads), 0, s, a,
              a_rs, wt, w_rs, bs, rs, r_rs, o, o_rs, M, N, K, 0.f, extra);
}

template <int STEPS, int NCOL>
void launch_lds_cols(const void* A, int64_t a_rs, const void* W, int64_t w_rs, const void* bias, const void* res,
                     int64_t r_rs, void* out, int64_t o_rs, int M, int N, int K, hipStream_t s) {
  const bf16_t *a = (const bf16_t*)A, *wt = (const bf16_t*)W, *bs = (const bf16_t*)bias, *rs = (const bf16_t*)res;
  bf16_t* o = (bf16_t*)out;
  if (bias && res)
    launch_lds_one<STEPS, true, true, NCOL>(a, a_rs, wt, w_rs, bs, rs, r_rs, o, o_rs, M, N, K, s);
  else if (bias)
    launch_lds_one<STEPS, true, false, NCOL>(a, a_rs, wt, w_rs, bs, rs, r_rs, o, o_rs, M, N, K, s);
  else if (res)
    launch_lds_one<STEPS, false, true, NCOL>(a, a_rs, wt, w_rs, bs, rs, r_rs, o, o_rs, M, N, K, s);
  else
    launch_lds_one<STEPS, false, false, NCOL>(a, a_rs, wt, w_rs, bs, rs, r_rs, o, o_rs, M, N, K, s);
}

template <int STEPS>
void launch_lds(const void* A, int64_t a_rs, const void* W, int64_t w_rs, const void* bias, const void* res,
                int64_t r_rs, void* out, int64_t o_rs, int M, int N, int K, hipStream_t s) {
  if (cols8(N))
    launch_lds_cols<STEPS, 8>(A, a_rs, W, w_rs, bias, res, r_rs, out, o_rs, M, N, K, s);
  else
    launch_lds_cols<STEPS, 16>(A, a_rs, W, w_rs, bias, res, r_rs, out, o_rs, M, N, K, s);
}

template <int STEPS>
void launch_steps(const void* A, int64_t a_rs, const void* W, int64_t w_rs, const void* bias, const void* res,
                  int64_t r_rs, void* out, int64_t o_rs, int M, int N, int K, hipStream_t s) {
  const dim3 grid((unsigned)((N + 15) / 16));
  const bf16_t *a = (const bf16_t*)A, *wt = (const bf16_t*)W, *bs = (const bf16_t*)bias, *rs = (const bf16_t*)res;
  bf16_t* o = (bf16_t*)out;
  if (bias && res)
    HDCM_LAUNCH((skinny_gemm_kernel<STEPS, true, true>), grid, dim3(kThreads), 0, s, a, a_rs, wt, w_rs, bs,
                       rs, r_rs, o, o_rs, M, N, K, 0.f);
  else if (bias)
    HDCM_LAUNCH((skinny_gemm_kernel<STEPS, true, false>), grid, dim3(kThreads), 0, s, a, a_rs, wt, w_rs,
                       bs, rs, r_rs, o, o_rs, M, N, K, 0.f);
  else if (res)
    HDCM_LAUNCH((skinny_gemm_kernel<STEPS, false, true>), grid, dim3(kThreads), 0, s, a, a_rs, wt, w_rs,
                       bs, rs, r_rs, o, o_rs, M, N, K, 0.f);
  else
    HDCM_LAUNCH((skinny_gemm_kernel<STEPS, false, false>), grid, dim3(kThreads), 0, s, a, a_rs, wt,
                       w_rs, bs, rs, r_rs, o, o_rs, M, N, K, 0.f);
}

template <int STEPS, bool WIDE>
void launch_ln(const bf16_t* c, int64_t c_rs, const bf16_t* W, int64_t w_rs, const bf16_t* res, int64_t r_rs,
               bf16_t* out, int64_t o_rs, int M, int N, int K, float eps, hipStream_t s) {
  const dim3 grid((unsigned)((N + 15) / 16));
  // narrow wide-kernel outputs (up to 4096 columns by default, e.g. the d_model 2048
  // out_proj): 8 columns per workgroup, so 2 workgroups per 16 columns stream the weight
  if constexpr (WIDE) {
    if (cols8(N))
      HDCM_LAUNCH((skinny_lds_kernel<STEPS, false, true, true, 8>), dim3((unsigned)((N + 7) / 8)),
                  dim3(kLdsThreads), 0, s, c, c_rs, W, w_rs, (const bf16_t*)nullptr, res, r_rs, out, o_rs, M, N, K,
                  eps, 0);
    else
      HDCM_LAUNCH((skinny_lds_kernel<STEPS, false, true, true>), grid, dim3(kLdsThreads), 0, s, c, c_rs, W,
                  w_rs, (const bf16_t*)nullptr, res, r_rs, out, o_rs, M, N, K, eps, 0);
  }
  else
    HDCM_LAUNCH((skinny_gemm_kernel<STEPS, false, true, true>), grid, dim3(kThreads), 0, s, c, c_rs, W,
                       w_rs, (const bf16_t*)nullptr, res, r_rs, out, o_rs, M, N, K, eps);
}

}  // namespace

// out = res + LN(c) W^T (row LayerNorm without affine over K) for M <= 16 rows: the skinny
// kernels with the fold above.  Called by hdcm_rowln_gemm_fwd after its argument checks.
bool hdcm_skinny_rowln_ok(int64_t M, int64_t K) {
  return M <= 16 && K % 32 == 0 && K <= (int64_t)kWaves * kMaxSteps * 32;
}
int hdcm_skinny_rowln(const void* c, int64_t c_rs, const void* W, int64_t w_rs, const void* res, int64_t r_rs,
                      void* out, int64_t o_rs, int64_t M, int64_t N, int64_t K, float eps, hipStream_t s) {
  const bool wide = N >= kWideN;
  const int steps = wide ? (int)((K / 32 + kLdsWaves - 1) / kLdsWaves) : (int)((K / 32 + kWaves - 1) / kWaves);
  const bf16_t *cc = (const bf16_t*)c, *ww = (const bf16_t*)W, *rr = (const bf16_t*)res;
  bf16_t* o = (bf16_t*)out;
  const int m = (int)M, n = (int)N, k = (int)K;
  if (wide) {
    if (steps <= 4) launch_ln<4, true>(cc, c_rs, ww, w_rs, rr, r_rs, o, o_rs, m, n, k, eps, s);
    else if (steps <= 8) launch_ln<8, true>(cc, c_rs, ww, w_rs, rr, r_rs, o, o_rs, m, n, k, eps, s);
    else if (steps <= 9) launch_ln<9, true>(cc, c_rs, ww, w_rs, rr, r_rs, o, o_rs, m, n, k, eps, s);
    else launch_ln<12, true>(cc, c_rs, ww, w_rs, rr, r_rs, o, o_rs, m, n, k, eps, s);
  } else {
    if (steps <= 8) launch_ln<8, false>(cc, c_rs, ww, w_rs, rr, r_rs, o, o_rs, m, n, k, eps, s);
    else if (steps <= 12) launch_ln<12, false>(cc, c_rs, ww, w_rs, rr, r_rs, o, o_rs, m, n, k, eps, s);
    else if (steps <= 18) launch_ln<18, false>(cc, c_rs, ww, w_rs, rr, r_rs, o, o_rs, m, n, k, eps, s);
    else launch_ln<kMaxSteps, false>(cc, c_rs, ww, w_rs, rr, r_rs, o, o_rs, m, n, k, eps, s);
  }
  return hdcm_launch_status();
}

extern "C" int hdcm_skinny_gemm_fwd(const void* A, int64_t a_row_stride, const void* W, int64_t w_row_stride,
                                    const void* bias, const void* res, int64_t res_row_stride, void* out,
                                    int64_t out_row_stride, int64_t M, int64_t N, int64_t K, int dtype,
                                    void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG((A || M == 0) && (W || N == 0) && (out || M == 0 || N == 0), HDCM_EINVAL);
  HDCM_CHECK_ARG(M >= 0 && N >= 0 && K > 0, HDCM_EINVAL);
  HDCM_CHECK_ARG(a_row_stride >= K && w_row_stride >= K && out_row_stride >= N, HDCM_EINVAL);
  HDCM_CHECK_ARG(!res || res_row_stride >= N, HDCM_EINVAL);
  HDCM_CHECK_ARG(M <= 16 && K % 32 == 0 && K <= (int64_t)kWaves * kMaxSteps * 32, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(N < ((int64_t)1 << 30), HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(hdcm_aligned16(A) && hdcm_aligned16(W) && a_row_stride % 8 == 0 && w_row_stride % 8 == 0,
                 HDCM_EALIGN);
  if (M == 0 || N == 0) return HDCM_OK;
  hipStream_t s = (hipStream_t)stream;
  const int m = (int)M, n = (int)N, k = (int)K;
  if (N >= kWideN) {
    const int lsteps = (int)((K / 32 + kLdsWaves - 1) / kLdsWaves);  // <= 12 since K <= 3072
    if (lsteps <= 4)
      launch_lds<4>(A, a_row_stride, W, w_row_stride, bias, res, res_row_stride, out, out_row_stride, m, n, k, s);
    else if (lsteps <= 8)
      launch_lds<8>(A, a_row_stride, W, w_row_stride, bias, res, res_row_stride, out, out_row_stride, m, n, k, s);
    else if (lsteps <= 9)
      launch_lds<9>(A, a_row_stride, W, w_row_stride, bias, res, res_row_stride, out, out_row_stride, m, n, k, s);
    else
      launch_lds<12>(A, a_row_stride, W, w_row_stride, bias, res, res_row_stride, out, out_row_stride, m, n, k, s);
    return hdcm_launch_status();
  }
  const int steps = (int)((K / 32 + kWaves - 1) / kWaves);
  if (steps <= 8)
    launch_steps<8>(A, a_row_stride, W, w_row_stride, bias, res, res_row_stride, out, out_row_stride, m, n, k, s);
  else if (steps <= 12)
    launch_steps<12>(A, a_row_stride, W, w_row_stride, bias, res, res_row_stride, out, out_row_stride, m, n, k, s);
  else if (steps <= 18)
    launch_steps<18>(A, a_row_stride, W, w_row_stride, bias, res, res_row_stride, out, out_row_stride, m, n, k, s);
  else
    launch_steps<kMaxSteps>(A, a_row_stride, W, w_row_stride, bias, res, res_row_stride, out, out_row_stride, m,
                            n, k, s);
  return hdcm_launch_status();
}

extern "C" size_t hdcm_step_workspace_bytes(void) { return kStepWsBytes; }

extern "C" int hdcm_norm_conv_in_proj_step_fwd(const void* x, int64_t x_row_stride, const void* ln_w,
                                               const void* ln_b, const void* conv_w, const void* conv_b, void* hist,
                                               float eps, void* u, int64_t u_row_stride, const void* W,
                                               int64_t w_row_stride, const void* bias, void* out,
                                               int64_t out_row_stride, int64_t B, int64_t D, int64_t N, void* ws,
                                               size_t ws_bytes, int dtype, void* stream) {
  HDCM_CHECK_ARG(dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(x && ln_w && ln_b && conv_w && conv_b && hist && u && W && out, HDCM_EINVAL);
  HDCM_CHECK_ARG(B >= 1 && D > 0 && N > 0, HDCM_EINVAL);
  HDCM_CHECK_ARG(x_row_stride >= D && u_row_stride >= D && w_row_stride >= D && out_row_stride >= N, HDCM_EINVAL);
  HDCM_CHECK_ARG(B <= kStepMaxRows && D % 32 == 0 && D <= 2048 && N < ((int64_t)1 << 30), HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(ws != nullptr && ws_bytes >= kStepWsBytes, HDCM_EWORKSPACE);
  HDCM_CHECK_ARG(((uintptr_t)ws & 127u) == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(hdcm_aligned16(x) && hdcm_aligned16(u) && hdcm_aligned16(hist) && hdcm_aligned16(ln_w) &&
                     hdcm_aligned16(ln_b) && hdcm_aligned16(conv_w) && hdcm_aligned16(conv_b) &&
                     hdcm_aligned16(W) && x_row_stride % 8 == 0 && u_row_stride % 8 == 0 &&
                     w_row_stride % 8 == 0,
                 HDCM_EALIGN);
  hipStream_t s = (hipStream_t)stream;
  const bf16_t *xx = (const bf16_t*)x, *lw = (const bf16_t*)ln_w, *lb = (const bf16_t*)ln_b,
               *cw = (const bf16_t*)conv_w, *cb = (const bf16_t*)conv_b, *ww = (const bf16_t*)W,
               *bs = (const bf16_t*)bias;
  bf16_t *hh = (bf16_t*)hist, *uu = (bf16_t*)u, *oo = (bf16_t*)out;
  unsigned* hdr = (unsigned*)ws;
  const int m = (int)B, n = (int)N, k = (int)D;
  const int lsteps = (k / 32 + kLdsWaves - 1) / kLdsWaves;  // <= 8 since D <= 2048
  if (lsteps <= 4)
    return launch_nc_in<4>(xx, x_row_stride, lw, lb, cw, cb, hh, eps, uu, u_row_stride, ww, w_row_stride, bs, oo,
                           out_row_stride, m, n, k, hdr, s);
  return launch_nc_in<8>(xx, x_row_stride, lw, lb, cw, cb, hh, eps, uu, u_row_stride, ww, w_row_stride, bs, oo,
                         out_row_stride, m, n, k, hdr, s);
}
