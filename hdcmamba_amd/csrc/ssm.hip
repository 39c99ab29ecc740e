// Diagonal selective scan over d_state channels for gfx950.
//
// Semantics (hdcmamba/model.py:175-233, intended form): per channel d and row t,
//   dt = softplus(dt_raw) with threshold 20 (log(1+exp(x)) below it),
//   a_t = exp(dt * A_d), A_d = -exp(A_log_d),  u_t = dt * b * x,
//   h_t = a_t * h_{t-1} + u_t,  y_t = h_t.
// All state is fp32; y is rounded once to the activation dtype.
//
// The recurrence is the associative scan of pairs (a, u) under
//   (a1, u1) then (a2, u2)  =  (a1*a2, a2*u1 + u2).
//
// Forward (ssm_scan_kernel): one launch that reads every input once.  A workgroup owns a
// tile of TR = 512 rows x 32 channels.  A thread holds one 16-byte channel group (8 bf16 or
// 4 fp32 channels) of 4 (bf16) or 8 (fp32) consecutive rows and
// scans them serially in registers; the row groups' totals are folded through LDS
// in sixteen segments, and the tile total (A, H) per channel is published after two barriers,
// before the row groups' prefixes within the tile are formed.  The workgroup then folds the
// totals of all earlier tiles of its sequence into the
// state entering the tile (decoupled look-back over totals, no inclusive chain), applies it
// to the rows it still holds in registers and stores y once.  Totals are published as 64-bit
// agent-scope atomic words {value, tag} that bypass the non-coherent per-XCD L2s, one word
// for A and one for H, so a reader needs no fence: a word is valid when its tag is this
// call's.  The tag is an epoch kept in the workspace header, read by every workgroup at its
// start; each workgroup then counts itself in one of eight counters of the header (an atomic
// whose latency hides behind its loads; the workgroup that completes a counter counts it in a
// ninth), and the last to arrive advances the epoch when it ends (every workgroup has read the
// tag by then, and nothing reads the header again in this call), so the workspace needs
// clearing only once, before its first use.  The tag and the counters sit on 128-byte lines of
// their own: one counter on the tag's line took every workgroup's arrival in turn, ~1 us of the
// scan at 256 workgroups.  A workgroup that finds an earlier total missing
// polls for a bounded number of rounds, then computes that tile's total itself with the
// same code and publishes it on the owner's behalf (identical bits), so no wait is unbounded
// whatever order the workgroups run in.  With row_stats the workgroup also writes, per row,
// the sum and the sum of squares of the 32 values it stored (as rounded), block-major (the
// rows of one channel block contiguous): the partial statistics of the row LayerNorm that
// follows, taken without another read of y.
//
// Backward (the adjoint scan, reversed rows): the three-pass form below.
//   1. ssm_tile_kernel<SUMMARY>: stage a tile's (a, u) pairs for 64 channels through LDS,
//      scan each channel with lanes = rows, keep the tile total (A, H) [b][channel][tile].
//   2. ssm_carry_kernel: per channel, scan the tile totals to get the state entering every
//      tile, h_in[b][channel][tile].
//   3. ssm_tile_kernel<OUTPUT>: rescan each tile, out_t = U_t + A_t * h_in, staged back
//      through LDS for 128-bit row stores.
#include <stdlib.h>

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

// ------------------------------------------------------------- single-pass forward
// 512 threads x (4 rows x 8 channels bf16, 8 rows x 4 channels fp32): 512-row tiles of 32
// channels, so a 32768-row sequence has
// 64 tiles and every look-back is one window of lanes = tiles.
constexpr int kScanThreads = 512;
constexpr int kScanCh = 32;  // channels per workgroup
constexpr int kScanWaves = kScanThreads / kWave;
// workspace header: the epoch (word 0), eight arrival counters and the count of completed
// counters, each on a 128-byte line of its own (words 32, 64, ..., 288)
constexpr int kHeaderBytes = 2048;
constexpr int kHdrLine = 32;     // u32 words per 128-byte line
constexpr int kArrivalGroups = 8;
constexpr int kBufferFlags = 0x00020000;  // buffer resource word 3: raw 32-bit dwords
constexpr int kCachePolicySC1 = 16;       // buffer load cache policy: agent-scope coherent (sc1)

template <typename T>
struct ScanShape {
  static constexpr int E = 16 / sizeof(T);      // channels per thread: one 16-byte group
  static constexpr int RPT = 32 / E;            // rows per thread (4 bf16, 8 fp32)
  static constexpr int CG = kScanCh / E;        // channel groups per tile
  static constexpr int RG = kScanThreads / CG;  // row groups per tile
  static constexpr int TR = RG * RPT;           // rows per tile: 512
};

// Largest tile count any dtype needs for L rows.
inline int64_t scan_tiles_max(int64_t L) { return (L + ScanShape<float>::TR - 1) / ScanShape<float>::TR; }

// A thread's channels of one row as stored: one 16-byte group.
template <typename T> struct ScanRawOf;
template <> struct ScanRawOf<bf16_t> { using type = uint4; };
template <> struct ScanRawOf<float> { using type = uint4; };
template <typename T> using ScanRaw = typename ScanRawOf<T>::type;
template <typename T> __device__ __forceinline__ ScanRaw<T> scan_ld(const T* p) {
  return *reinterpret_cast<const ScanRaw<T>*>(p);
}
template <typename T>
__device__ __forceinline__ void scan_unpack(ScanRaw<T> v, float (&o)[ScanShape<T>::E]) {
  unpack16<T>(v, o);
}

// Workspace layout: header (epoch, arrival counters), then the tile totals: per
// sequence (batch row x channel block), channel and tile one 16-byte (A, H) pair of tagged
// words.
struct ScanWorkspace {
  int64_t words_at, words_bytes;
};
inline ScanWorkspace scan_workspace(int64_t B, int64_t L, int64_t ds) {
  const int64_t nseq = B * ((ds + kScanCh - 1) / kScanCh);
  ScanWorkspace w;
  w.words_at = kHeaderBytes;
  w.words_bytes = nseq * kScanCh * scan_tiles_max(L) * 16;
  return w;
}

__device__ __forceinline__ unsigned long long pack_word(float v, unsigned tag) {
  return ((unsigned long long)tag << 32) | (unsigned long long)__float_as_uint(v);
}
__device__ __forceinline__ float word_value(unsigned long long w) { return __uint_as_float((unsigned)w); }
__device__ __forceinline__ unsigned word_tag(unsigned long long w) { return (unsigned)(w >> 32); }

// Row r (< RPT) of this thread's rows of a tile (tile*TR + rg*RPT + r, clamped to L-1:
// rows past L are re-read and masked later) at its channel group (group 0 past nch).
template <typename T>
__device__ __forceinline__ const T* row_ptr(const T* __restrict__ projs, int64_t prs, int64_t rowbase, int tile,
                                            int c0, int nch, int L, int r) {
  using S = ScanShape<T>;
  const int tid = threadIdx.x, cg = tid % S::CG, rg = tid / S::CG;
  const int t = min(tile * S::TR + rg * ScanShape<T>::RPT + r, L - 1);
  return projs + (rowbase + t) * prs + (cg * S::E < nch ? c0 + cg * S::E : 0);
}

// This thread's rows x E channels of dt, x, b, as stored: every thread issues the same
// 3*RPT loads.
template <typename T>
__device__ __forceinline__ void load_rows(const T* __restrict__ projs, int64_t prs, int64_t rowbase, int tile, int c0,
                                          int nch, int L, int ds, ScanRaw<T> (&raw)[ScanShape<T>::RPT][3]) {
#pragma unroll
  for (int r = 0; r < ScanShape<T>::RPT; ++r) {
    const T* p = row_ptr<T>(projs, prs, rowbase, tile, c0, nch, L, r);
    raw[r][0] = scan_ld<T>(p);
    raw[r][1] = scan_ld<T>(p + ds);
    raw[r][2] = scan_ld<T>(p + 2 * ds);
  }
}

// The pairs (a, u) of one row from its dt, x, b groups; the identity (1, 0) when !ok (rows
// past L, channels past nch).
template <typename T>
__device__ __forceinline__ void pairs_of(const ScanRaw<T> (&g)[3], const float (&negA)[ScanShape<T>::E], bool ok,
                                         float (&a)[ScanShape<T>::E], float (&u)[ScanShape<T>::E]) {
  constexpr int E = ScanShape<T>::E;
  float d[E], xv[E], bv[E];
  scan_unpack<T>(g[0], d);
  scan_unpack<T>(g[1], xv);
  scan_unpack<T>(g[2], bv);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float dt = softplus20(d[e]);
    a[e] = ok ? fexp(dt * negA[e]) : 1.f;
    u[e] = ok ? (dt * bv[e]) * xv[e] : 0.f;
  }
}

// One row folded into this thread's running total (ca, ch), rows in order.  Every
// multiply-add here and in combine_total is an explicit fmaf, so a tile total has identical
// bits wherever it is computed (by the tile's owner, or by a workgroup computing it on the
// owner's behalf with tile_total_streamed).
template <typename T>
__device__ __forceinline__ void fold_row(const ScanRaw<T> (&g)[3], const float (&negA)[ScanShape<T>::E], bool ok,
                                         float (&ca)[ScanShape<T>::E], float (&ch)[ScanShape<T>::E]) {
  constexpr int E = ScanShape<T>::E;
  float a[E], u[E];
  pairs_of<T>(g, negA, ok, a, u);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    ch[e] = fmaf(a[e], ch[e], u[e]);
    ca[e] = ca[e] * a[e];
  }
}

// LDS of the cross-thread part of a tile: one (A, H) pair per channel and row group, stored
// channel-major with an odd pitch (the threads of a segment read 32 consecutive channels of
// one row group, and the threads of a row group write their channels, on distinct banks), and
// the segment totals.
constexpr int kMaxRG = kScanThreads / (kScanCh / 8);  // row groups of a tile (bf16: the most)
constexpr int kSeg = kScanThreads / kScanCh;          // row-group segments, one thread per channel each
constexpr int kRGPitch = kMaxRG + 1;
struct ScanLds {
  float rgA[kScanCh][kRGPitch];
  float rgH[kScanCh][kRGPitch];
  float seg[kSeg][kScanCh][2];
};

// The tile total from each thread's total (ca, ch) over its rows: the row groups' pairs go to
// LDS, thread (segment s, channel c) folds its run of RGS row groups in order (kept in va, vh
// for combine_prefix), and the threads of segment 0 (tid < 32, channel tid) fold the segment
// totals in order into (tA, tH).  Two barriers.
template <typename T>
__device__ __forceinline__ void combine_total(const float (&ca)[ScanShape<T>::E], const float (&ch)[ScanShape<T>::E],
                                              float (&va)[ScanShape<T>::RG / kSeg],
                                              float (&vh)[ScanShape<T>::RG / kSeg], float& tA, float& tH,
                                              ScanLds* lds) {
  using S = ScanShape<T>;
  constexpr int E = S::E, CG = S::CG, RG = S::RG;
  constexpr int RGS = RG / kSeg;  // row groups per segment
  static_assert(RG % kSeg == 0 && RG <= kMaxRG, "row-group segments");
  const int tid = threadIdx.x, cg = tid % CG, rg = tid / CG;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    lds->rgA[cg * E + e][rg] = ca[e];
    lds->rgH[cg * E + e][rg] = ch[e];
  }
  __syncthreads();
  const int c = tid % kScanCh, s = tid / kScanCh;
  float sa = 1.f, sh = 0.f;
#pragma unroll
  for (int k = 0; k < RGS; ++k) {
    va[k] = lds->rgA[c][s * RGS + k];
    vh[k] = lds->rgH[c][s * RGS + k];
  }
#pragma unroll
  for (int k = 0; k < RGS; ++k) {
    sh = fmaf(va[k], sh, vh[k]);
    sa = sa * va[k];
  }
  lds->seg[s][c][0] = sa;
  lds->seg[s][c][1] = sh;
  __syncthreads();
  tA = 1.f, tH = 0.f;
  if (s == 0) {
#pragma unroll
    for (int k = 0; k < kSeg; ++k) {
      const float ka = lds->seg[k][c][0], kh = lds->seg[k][c][1];
      tH = fmaf(ka, tH, kh);
      tA = tA * ka;
    }
  }
}

// After combine_total (same va, vh): each row group's exclusive prefix within the tile, handed
// back to its threads as (xa, xh) for their E channels.  Two barriers; the LDS is free after.
template <typename T>
__device__ __forceinline__ void combine_prefix(const float (&va)[ScanShape<T>::RG / kSeg],
                                               const float (&vh)[ScanShape<T>::RG / kSeg], float (&xa)[ScanShape<T>::E],
                                               float (&xh)[ScanShape<T>::E], ScanLds* lds) {
  using S = ScanShape<T>;
  constexpr int E = S::E, CG = S::CG, RGS = S::RG / kSeg;
  const int tid = threadIdx.x;
  const int c = tid % kScanCh, s = tid / kScanCh;
  float pa = 1.f, ph = 0.f;  // segments before s
  for (int k = 0; k < s; ++k) {
    const float ka = lds->seg[k][c][0], kh = lds->seg[k][c][1];
    ph = fmaf(ka, ph, kh);
    pa = pa * ka;
  }
#pragma unroll
  for (int k = 0; k < RGS; ++k) {
    lds->rgA[c][s * RGS + k] = pa;
    lds->rgH[c][s * RGS + k] = ph;
    ph = fmaf(va[k], ph, vh[k]);
    pa = pa * va[k];
  }
  __syncthreads();
  const int cg = tid % CG, rg = tid / CG;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    xa[e] = lds->rgA[cg * E + e][rg];
    xh[e] = lds->rgH[cg * E + e][rg];
  }
  __syncthreads();  // the LDS is reused
}

// A tile's total (threads tid < 32: channel tid) with the rows read one at a time (few
// registers in use): the kernel's own fold, row by row in the same order, then
// combine_total, hence the same bits.
template <typename T>
__device__ __forceinline__ void tile_total_streamed(const T* __restrict__ projs, int64_t prs, int64_t rowbase,
                                                    int tile, int c0, int nch, int L, int ds,
                                                    const float (&negA)[ScanShape<T>::E], float& tA, float& tH,
                                                    ScanLds* lds) {
  using S = ScanShape<T>;
  constexpr int E = S::E;
  const int tid = threadIdx.x, cg = tid % S::CG, rg = tid / S::CG;
  const bool cok = cg * E < nch;
  const int r0 = tile * S::TR + rg * ScanShape<T>::RPT;
  float ca[E], ch[E];
#pragma unroll
  for (int e = 0; e < E; ++e) ca[e] = 1.f, ch[e] = 0.f;
#pragma unroll 1
  for (int r = 0; r < ScanShape<T>::RPT; ++r) {
    const T* p = row_ptr<T>(projs, prs, rowbase, tile, c0, nch, L, r);
    const ScanRaw<T> g[3] = {scan_ld<T>(p), scan_ld<T>(p + ds), scan_ld<T>(p + 2 * ds)};
    fold_row<T>(g, negA, cok && r0 + r < L, ca, ch);
  }
  float va[S::RG / kSeg], vh[S::RG / kSeg];
  combine_total<T>(ca, ch, va, vh, tA, tH, lds);
  __syncthreads();  // the LDS is reused
}

// The tile total of channel tid (< 32), published for later tiles.
__device__ __forceinline__ void publish_total(unsigned long long* words, int64_t seq, int ntiles, int tile,
                                              int nch, float tA, float tH, unsigned tag) {
  const int c = threadIdx.x;
  if (c >= nch) return;  // also every thread past the first 32 (nch <= 32)
  unsigned long long* p = words + 2 * ((seq * kScanCh + c) * ntiles + tile);
  __hip_atomic_store(p, pack_word(tA, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(p + 1, pack_word(tH, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Compute and publish, with this call's tag, the totals of the tiles j0 + k for the set bits
// k of `missing` (the rare path of the look-back), and keep them in fill[k][channel] for the
// caller's own fold.  All threads of the workgroup call it together.
template <typename T>
__device__ __forceinline__ void publish_missing(const T* __restrict__ projs, int64_t prs,
                                                const float (&negA)[ScanShape<T>::E], unsigned long long* words, int64_t seq,
                                                int64_t rowbase, int c0, int nch, int L, int ds, int ntiles, int j0,
                                                unsigned long long missing, unsigned tag, ScanLds* lds,
                                                float (*fill)[kScanCh][2]) {
  while (missing != 0) {
    const int k = __builtin_ctzll(missing);
    const int jm = j0 + k;
    missing &= missing - 1;
    float tA, tH;
    tile_total_streamed<T>(projs, prs, rowbase, jm, c0, nch, L, ds, negA, tA, tH, lds);
    publish_total(words, seq, ntiles, jm, nch, tA, tH, tag);
    if (threadIdx.x < kScanCh) {
      fill[k][threadIdx.x][0] = tA;
      fill[k][threadIdx.x][1] = tH;
    }
  }
}

// One workgroup per (tile, 32-channel block, sequence).  See the file header.
template <typename T>
__global__ __launch_bounds__(kScanThreads) void ssm_scan_kernel(
    const T* __restrict__ projs, int64_t prs, const T* __restrict__ A_log, const float* __restrict__ h0,
    T* __restrict__ y, int64_t yrs, float* __restrict__ h_final, float* __restrict__ row_stats, int64_t stats_ps,
    unsigned* __restrict__ hdr, unsigned long long* __restrict__ words, int words_bytes, int L, int ds, int ntiles,
    int spin_rounds) {
  using S = ScanShape<T>;
  constexpr int E = S::E, CG = S::CG;
  constexpr int CPW = kScanCh / kScanWaves;  // look-back channels per wave
  __shared__ ScanLds s_lds;
  __shared__ float s_hin[kScanCh];
  __shared__ unsigned s_missing[kScanWaves][2];
  __shared__ float s_fill[kWave][kScanCh][2];  // totals this workgroup computed for a window
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int cg = tid % CG, rg = tid / CG;
  const int tile = blockIdx.x, chb = blockIdx.y, b = blockIdx.z;
  const int c0 = chb * kScanCh;
  const int nch = min(kScanCh, ds - c0);
  const bool cok = cg * E < nch;
  const int64_t seq = (int64_t)b * gridDim.y + chb;  // this tile's sequence of totals
  const int64_t rowbase = (int64_t)b * L;
  // Loads in this order, none waited for before the next is issued: the call's tag, this
  // thread's A_log group, then every row of the tile; the tag and A_log (the oldest) are
  // back before the first row, so the fold below takes the rows as they arrive.
  const unsigned tag = __hip_atomic_load(hdr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  ScanRaw<T> araw{};
  if (cok) araw = scan_ld<T>(A_log + c0 + cg * E);
  ScanRaw<T> raw[ScanShape<T>::RPT][3];
  load_rows<T>(projs, prs, rowbase, tile, c0, nch, L, ds, raw);
  // Arrival count, issued once the tag has been read (the asm needs its value), so the last
  // arrival knows that every workgroup of the call has read it.  The address goes through a
  // register the compiler cannot see into, which keeps the atomic as one lane's operation
  // whose result is waited for only at the end (not reduced across the wave on the spot).
  unsigned arrived = 0;
  if (tid == 0) {
    unsigned zero;
    __asm__ volatile("v_mov_b32 %0, 0" : "=v"(zero) : "v"(tag));
    const unsigned lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    arrived = __hip_atomic_fetch_add(hdr + kHdrLine * (1 + lin % kArrivalGroups) + zero, 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
  }

  float negA[E];
  {
    float al[E];
    scan_unpack<T>(araw, al);
#pragma unroll
    for (int e = 0; e < E; ++e) negA[e] = -fexp(al[e]);
  }
  // this thread's rows: the prefixes (At, Ut) of its own rows, kept for the outputs, then the
  // tile's exclusive prefix and total
  float At[S::RPT][E], Ut[S::RPT][E], xa[E], xh[E];
  float va[S::RG / kSeg], vh[S::RG / kSeg], tA, tH;
  {
    const int r0 = tile * S::TR + rg * ScanShape<T>::RPT;
    float ca[E], ch[E];
#pragma unroll
    for (int e = 0; e < E; ++e) ca[e] = 1.f, ch[e] = 0.f;
#pragma unroll
    for (int r = 0; r < ScanShape<T>::RPT; ++r) {
      fold_row<T>(raw[r], negA, cok && r0 + r < L, ca, ch);
#pragma unroll
      for (int e = 0; e < E; ++e) At[r][e] = ca[e], Ut[r][e] = ch[e];
    }
    combine_total<T>(ca, ch, va, vh, tA, tH, &s_lds);
  }
  publish_total(words, seq, ntiles, tile, nch, tA, tH, tag);
  combine_prefix<T>(va, vh, xa, xh, &s_lds);  // off the critical path: the stores are in flight
  const __amdgpu_buffer_rsrc_t wrsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)words, (short)0, words_bytes, kBufferFlags);

  // ---- state entering this tile: fold the totals of tiles 0 .. tile-1 (lanes = tiles, 64 at a
  // time; wave w folds channels w*CPW .. +CPW-1), then apply to h0
  float fa[CPW], fh[CPW];
#pragma unroll
  for (int k = 0; k < CPW; ++k) fa[k] = 1.f, fh[k] = 0.f;
  // the (A, H) words of tile j0 + lane for this wave's channels: 16 bytes each, read through
  // the buffer path with the agent-scope cache policy (coalesced, and never a stale L2 line;
  // each 8-byte half carries its own tag, so a read torn between two stores shows a stale
  // half and is read again)
  // (lanes with `again` false keep what they hold: after the first round only the tiles some
  // wave still missed are read again)
  auto read_window = [&](int j0, uint4 (&q)[CPW], bool again) {
    const int j = j0 + lane;
#pragma unroll
    for (int k = 0; k < CPW; ++k) {
      const int c = w * CPW + k;
      if (j < tile && c < nch) {
        if (again)
          q[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                               wrsrc, (int)(((seq * kScanCh + c) * ntiles + j) * 16), 0,
                                               kCachePolicySC1));
      } else {
        q[k] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  for (int j0 = 0; j0 < tile; j0 += kWave) {
    const int j = j0 + lane;
    const bool act = j < tile;
    uint4 q[CPW];
    float va[CPW], vh[CPW];
    unsigned long long all = ~0ull;  // tiles of the window to read: all of them, then the missed ones
    for (int round = 0;; ++round) {
      read_window(j0, q, (all >> lane) & 1ull);
      bool ok = true;
#pragma unroll
      for (int k = 0; k < CPW; ++k) {
        const int c = w * CPW + k;
        va[k] = 1.f, vh[k] = 0.f;
        if (act && c < nch) {
          const unsigned long long wa = ((unsigned long long)q[k].y << 32) | q[k].x;
          const unsigned long long wh = ((unsigned long long)q[k].w << 32) | q[k].z;
          ok = ok && word_tag(wa) == tag && word_tag(wh) == tag;
          va[k] = word_value(wa);
          vh[k] = word_value(wh);
        }
      }
      // tiles of this window that some wave still misses (one bit per lane)
      const unsigned long long miss = __ballot(!ok);
      if (lane == 0) {
        s_missing[w][0] = (unsigned)miss;
        s_missing[w][1] = (unsigned)(miss >> 32);
      }
      __syncthreads();
      all = 0;
#pragma unroll
      for (int k = 0; k < kScanWaves; ++k)
        all |= (unsigned long long)s_missing[k][0] | ((unsigned long long)s_missing[k][1] << 32);
      __syncthreads();
      if (all == 0) break;
      if (round < spin_rounds) {
        __builtin_amdgcn_s_sleep(1);
        continue;
      }
      // still missing after the polling budget: compute those tiles' totals here, publish
      // them for their owners (the owner's own store later writes the same bits) and fold
      // the values computed here for them; every other tile of the window was read with
      // this call's tag by every wave.  No further read, so the loop ends here.
      publish_missing<T>(projs, prs, negA, words, seq, rowbase, c0, nch, L, ds, ntiles, j0, all, tag, &s_lds,
                         s_fill);
      __syncthreads();
      if (act && ((all >> lane) & 1ull)) {
#pragma unroll
        for (int k = 0; k < CPW; ++k) {
          const int c = w * CPW + k;
          if (c < nch) {
            va[k] = s_fill[lane][c][0];
            vh[k] = s_fill[lane][c][1];
          }
        }
      }
      break;
    }
    // fold this window in tile order: inclusive lane scan, the total sits in lane 63
    scan_pairs<CPW>(va, vh);
#pragma unroll
    for (int k = 0; k < CPW; ++k) {
      const float wa = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(va[k]), kWave - 1));
      const float wh = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vh[k]), kWave - 1));
      fh[k] = fmaf(wa, fh[k], wh);
      fa[k] = fa[k] * wa;
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < CPW; ++k) {
      const int c = w * CPW + k;
      const float hz = (h0 != nullptr && c < nch) ? h0[(int64_t)b * ds + c0 + c] : 0.f;
      s_hin[c] = fmaf(fa[k], hz, fh[k]);
    }
  }
  __syncthreads();

  // ---- outputs: y_t = U_t + A_t * (state entering this thread's rows)
  const int r0 = tile * S::TR + rg * ScanShape<T>::RPT;
  float hs[E];
#pragma unroll
  for (int e = 0; e < E; ++e) hs[e] = fmaf(xa[e], s_hin[cg * E + e], xh[e]);
  float rsum[S::RPT], rsq[S::RPT];  // this thread's part of each row's sum and sum of squares
  if (cok) {
    T* yb = y + rowbase * yrs + c0 + cg * E;
#pragma unroll
    for (int r = 0; r < ScanShape<T>::RPT; ++r) {
      const int t = r0 + r;
      rsum[r] = rsq[r] = 0.f;
      if (t >= L) continue;
      float v[E];
#pragma unroll
      for (int e = 0; e < E; ++e) v[e] = fmaf(At[r][e], hs[e], Ut[r][e]);
      store16_sums<T>(yb + (int64_t)t * yrs, v, rsum[r], rsq[r]);
      if (h_final != nullptr && t == L - 1) {
#pragma unroll
        for (int e = 0; e < E; ++e) h_final[(int64_t)b * ds + c0 + cg * E + e] = v[e];
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < ScanShape<T>::RPT; ++r) rsum[r] = rsq[r] = 0.f;
  }
  if (row_stats != nullptr) {  // the CG threads of a row group are consecutive lanes
#pragma unroll
    for (int r = 0; r < ScanShape<T>::RPT; ++r) {
      const float s = group_sum<CG>(rsum[r]), q = group_sum<CG>(rsq[r]);
      const int t = r0 + r;
      if (cg == 0 && t < L)
        *reinterpret_cast<float2*>(row_stats + 2 * (chb * stats_ps + rowbase + t)) = make_float2(s, q);
    }
  }

  // ---- the workgroup that completes its counter counts it in the last one; the one that
  // completes that advances the epoch and clears the counters for the next call
  if (tid == 0) {
    const unsigned G = gridDim.x * gridDim.y * gridDim.z;
    const unsigned x = (blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)) % kArrivalGroups;
    if (arrived == (G - x + kArrivalGroups - 1) / kArrivalGroups - 1) {
      unsigned* done = hdr + kHdrLine * (1 + kArrivalGroups);
      const unsigned groups = G < (unsigned)kArrivalGroups ? G : (unsigned)kArrivalGroups;
      if (__hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == groups - 1) {
        for (int k = 0; k < kArrivalGroups; ++k)
          __hip_atomic_store(hdr + kHdrLine * (1 + k), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(hdr, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// polling rounds before a missing total is computed here (HDCM_OPT_SSM_SPIN_ROUNDS; 0 forces
// the compute-it-here path, a test hook)
int spin_rounds_setting() { return hdcm_option_value(HDCM_OPT_SSM_SPIN_ROUNDS); }

template <typename T>
int launch(const void* projs, int64_t prs, const void* A_log, const float* h0, void* y,
           int64_t yrs, float* h_final, float* row_stats, int64_t stats_ps, void* ws, int64_t B, int64_t L,
           int64_t ds, hipStream_t s) {
  const int64_t nt = (L + ScanShape<T>::TR - 1) / ScanShape<T>::TR;
  const dim3 grid((unsigned)nt, (unsigned)((ds + kScanCh - 1) / kScanCh), (unsigned)B);
  const ScanWorkspace w = scan_workspace(B, L, ds);
  char* base = (char*)ws;
  HDCM_LAUNCH((ssm_scan_kernel<T>), grid, dim3(kScanThreads), 0, s, (const T*)projs, prs, (const T*)A_log, h0, (T*)y,
              yrs, h_final, row_stats, stats_ps, (unsigned*)base, (unsigned long long*)(base + w.words_at),
              (int)w.words_bytes, (int)L,
              (int)ds, (int)nt, spin_rounds_setting());
  return hdcm_launch_status();
}

}  // namespace

extern "C" size_t hdcm_ssm_workspace_bytes(int64_t B, int64_t L, int64_t ds) {
  if (B <= 0 || L <= 0 || ds <= 0) return 0;
  const ScanWorkspace w = scan_workspace(B, L, ds);
  return (size_t)(w.words_at + w.words_bytes);
}

// Argument checks of the forward entry points, everything but the workspace (also used by
// other sources of the library that run these kernels).
int hdcm_ssm_check_fwd(const void* projs, int64_t proj_row_stride, const void* A_log, const void* y,
                       int64_t y_row_stride, const float* row_stats, int64_t stats_part_stride, int64_t B,
                       int64_t L, int64_t ds, int dtype) {
  HDCM_CHECK_ARG(dtype == HDCM_F32 || dtype == HDCM_BF16, HDCM_EUNSUPPORTED);
  HDCM_CHECK_ARG(A_log && ((projs && y) || B == 0 || L == 0), HDCM_EINVAL);  // empty: NULL data allowed
  HDCM_CHECK_ARG(B >= 0 && L >= 0 && ds > 0, HDCM_EINVAL);
  HDCM_CHECK_ARG(proj_row_stride >= 3 * ds && y_row_stride >= ds, HDCM_EINVAL);
  const int E = 16 / hdcm_elt_size(dtype);
  HDCM_CHECK_ARG(ds % E == 0 && proj_row_stride % E == 0 && y_row_stride % E == 0, HDCM_EALIGN);
  HDCM_CHECK_ARG(hdcm_aligned16(projs) && hdcm_aligned16(y) && hdcm_aligned16(A_log), HDCM_EALIGN);
  HDCM_CHECK_ARG(B <= 65535 && ds <= 65535 && L < ((int64_t)1 << 30), HDCM_EUNSUPPORTED);
  // row_stats: one (sum, sum of squares) pair per 32-channel block and row, block-major
  HDCM_CHECK_ARG(!row_stats || stats_part_stride >= B * L, HDCM_EINVAL);
  HDCM_CHECK_ARG(((uintptr_t)row_stats & 7u) == 0, HDCM_EALIGN);
  // the scan kernel counts its workgroups, and addresses its tile totals, in 32 bits
  HDCM_CHECK_ARG(B * ((ds + kScanCh - 1) / kScanCh) * scan_tiles_max(L) < ((int64_t)1 << 31) / (kScanCh * 16),
                 HDCM_EUNSUPPORTED);
  return HDCM_OK;
}

// The forward's launch on a checked, non-empty input with a workspace of
// hdcm_ssm_workspace_bytes(B, L, ds) bytes at `ws` (256-byte aligned, zero before its first
// use, then left as the previous call left it).
int hdcm_ssm_launch_fwd(const void* projs, int64_t proj_row_stride, const void* A_log, const float* h0, void* y,
                        int64_t y_row_stride, float* h_final, float* row_stats, int64_t stats_part_stride, void* ws,
                        int64_t B, int64_t L, int64_t ds, int dtype, hipStream_t s) {
  if (dtype == HDCM_F32)
    return launch<float>(projs, proj_row_stride, A_log, h0, y, y_row_stride, h_final, row_stats, stats_part_stride,
                         ws, B, L, ds, s);
  return launch<bf16_t>(projs, proj_row_stride, A_log, h0, y, y_row_stride, h_final, row_stats, stats_part_stride,
                        ws, B, L, ds, s);
}

extern "C" int hdcm_ssm_fwd(const void* projs, int64_t proj_row_stride, const void* A_log,
                            const float* h0, void* y, int64_t y_row_stride, float* h_final,
                            float* row_stats, int64_t stats_part_stride, void* ws, size_t ws_bytes, int64_t B,
                            int64_t L, int64_t ds, int dtype, void* stream) {
  const int st = hdcm_ssm_check_fwd(projs, proj_row_stride, A_log, y, y_row_stride, row_stats, stats_part_stride, B,
                                    L, ds, dtype);
  if (st) return st;
  if (B == 0 || L == 0) return HDCM_OK;
  HDCM_CHECK_ARG(ws != nullptr && ws_bytes >= hdcm_ssm_workspace_bytes(B, L, ds), HDCM_EWORKSPACE);
  HDCM_CHECK_ARG(((uintptr_t)ws & 255u) == 0, HDCM_EALIGN);
  return hdcm_ssm_launch_fwd(projs, proj_row_stride, A_log, h0, y, y_row_stride, h_final, row_stats,
                             stats_part_stride, ws, B, L, ds, dtype, (hipStream_t)stream);
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
