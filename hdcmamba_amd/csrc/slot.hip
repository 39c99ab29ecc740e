// Slot memory (per-head decayed linear attention) fused with the per-token GroupNorm
// and sigmoid gate, for gfx950.
//
// Semantics (hdcmamba/model.py:236-272 and 274-293, intended form): for head h with
// decay gamma and feature map phi(z) = z+1 (z>0) else exp(z),
//   y_t = sum_{j<=t} w(t,j) (phi(q_t).phi(k_j)) v_j,
//   w(t,j) = gamma^(t-j) if j is in t's chunk of C rows, else gamma^(t-j-1);
//   out_t = GN_hd(y_t) * sigmoid(gate_t), GN over the head's hd values with affine.
// In bf16 the MFMA operands are rounded where the reference rounds its tl.dot
// operands: phi(q), phi(k), the decayed masked scores, phi(q)*gamma^c, the carried
// state and phi(k)*gamma^(C-1-c); accumulation is fp32.
//
// Decomposition.  Rows are processed in tiles of TC (64 for bf16, 32 for fp32).  Let p
// be a tile start and cs the start of p's chunk.  Two fp32 states are carried:
//   A = sum_{j<cs}     gamma^(cs-1-j) k~_j^T v_j      (the reference's `running`)
//   W = sum_{cs<=j<p}  gamma^(p-1-j)  k~_j^T v_j      (only when C > TC)
// and for t in the tile  y_t = intra_t + gamma^(t-p) phi(q_t) . S_eff,
//   S_eff = gamma*W + gamma^(p-cs)*A.
// When C divides TC every tile start is a chunk boundary (W = 0) and the cross-chunk
// factor gamma^-1 appears inside the tile's score matrix instead.
//
// Parallelism: the sequence is cut into segments of seg_tiles tiles that start on chunk
// boundaries.  slot_state_kernel computes each segment's contribution U_s to A (from k
// and v only), slot_scan_kernel turns them into the state at every segment start, and
// slot_gate_kernel walks each (batch, head, segment) with its own start state.  That
// gives B*H*nseg workgroups instead of the reference's B*H serial programs.
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16; fp32 uses 8x v_mfma_f32_16x16x4f32).  A C/D
// tile puts column n = lane%16 and rows 4*(lane/16)+r in a lane.  Scores are computed
// transposed, S^T[j][i] = phi(K) phi(Q)^T, so a lane holds one query column i and 4+4
// key rows j of two adjacent 16-row tiles; those 8 values are exactly a B-operand
// fragment of P^T for Y^T = V^T P^T under the slot permutation
//   slot s -> j = 32t + (s<4 ? 4g+s : 16+4g+s-4),  g = lane/16,
// applied identically to the V^T A-operand (two 8-byte LDS reads).  Y^T then leaves
// each lane one token row with 4 consecutive value columns per 16-column tile, so the
// GroupNorm needs only an in-lane sum and two cross-lane shuffles, and stores are
// contiguous runs of 4 elements.  The state update S[dk][dv] += K~^T V is split across
// the 4 waves by 16-column dv tiles and stays in MFMA accumulators; the rounded S_eff^T
// is shared through a double-buffered LDS tile.
#include <stdlib.h>

#include "hdcm_common.h"

using namespace hdcm;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kTargetWorkgroups = 2048;
constexpr int kMinSegTiles = 4;

template <typename T>
struct TileOf {
  static constexpr int value = sizeof(T) == 2 ? 64 : 32;
};

template <typename T, int HD, int TC>
struct Lds {
  static constexpr int PADE = 16 / sizeof(T);
  static constexpr int PR = HD + PADE;  // pitch of [TC][HD] row tiles and of [HD][HD] S^T
  static constexpr int PT = TC + PADE;  // pitch of transposed [HD][TC] tiles
  static constexpr int tileR = TC * PR;
  static constexpr int tileT = HD * PT;
  static constexpr int tileS = HD * PR;
  static constexpr int oQ = 0;            // phi(q)            [TC][HD]
  static constexpr int oQd = oQ + tileR;  // phi(q)*gamma^i    [TC][HD]
  static constexpr int oK = oQd + tileR;  // phi(k)            [TC][HD]
  static constexpr int oG = oK + tileR;   // gate (raw)        [TC][HD]
  static constexpr int oKt = oG + tileR;  // (phi(k)*decay)^T  [HD][TC]
  static constexpr int oVt = oKt + tileT; // v^T               [HD][TC]
  static constexpr int oS0 = oVt + tileT; // S_eff^T buffers   [HD][HD] x2
  static constexpr int oS1 = oS0 + tileS;
  static constexpr int total = oS1 + tileS;
  // state pre-pass uses only the two transposed tiles
  static constexpr int stKt = 0;
  static constexpr int stVt = tileT;
  static constexpr int stTotal = 2 * tileT;
};

__device__ __forceinline__ float phi_f(float z) { return z > 0.f ? z + 1.0f : expf(z); }

template <typename T>
__device__ __forceinline__ void store4(T* p, const float* v);
template <>
__device__ __forceinline__ void store4<float>(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
template <>
__device__ __forceinline__ void store4<bf16_t>(bf16_t* p, const float* v) {
  uint2 u;
  u.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
  u.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
  *reinterpret_cast<uint2*>(p) = u;
}

// Raw element e of a 16-byte group, as the storage type.
template <typename T>
__device__ __forceinline__ T raw_elem(const uint4& v, int e);
template <>
__device__ __forceinline__ float raw_elem<float>(const uint4& v, int e) {
  const uint32_t w = e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
  return __uint_as_float(w);
}
template <>
__device__ __forceinline__ bf16_t raw_elem<bf16_t>(const uint4& v, int e) {
  const uint32_t w = (e >> 1) == 0 ? v.x : (e >> 1) == 1 ? v.y : (e >> 1) == 2 ? v.z : v.w;
  return (bf16_t)((e & 1) ? (w >> 16) : (w & 0xffffu));
}

// Load the 16-byte groups of one tile owned by this thread.  Blocks are numbered
// q=0, k=1, v=2, gate=3; the thread covers blocks [B0, B0+NB).  Each tile block has
// TC*GPR groups, a multiple of kThreads, so the block of iteration `it` is uniform.
template <typename T, int HD, int TC, int B0, int NB>
__device__ __forceinline__ void load_tile(uint4 (&raw)[NB * HD / 32], const T* __restrict__ projs,
                                          int64_t prs, int64_t rowbase, int colbase, int dm, int p,
                                          int L, int tid) {
  constexpr int E = Vec<T>::N;
  constexpr int GPR = HD / E;
  constexpr int NL = NB * HD / 32;
  static_assert((TC * GPR) % kThreads == 0, "tile block must be a multiple of the workgroup");
  static_assert(NL * kThreads == NB * TC * GPR, "load count");
#pragma unroll
  for (int it = 0; it < NL; ++it) {
    const int idx = tid + kThreads * it;
    const int blk = B0 + (kThreads * it) / (TC * GPR);
    const int rem = idx % (TC * GPR);
    const int i = rem / GPR, cg = rem % GPR;
    raw[it] = (p + i < L)
                  ? ldg16(projs + (rowbase + p + i) * prs + colbase + blk * dm + cg * E)
                  : make_uint4(0, 0, 0, 0);
  }
}

// Write a loaded tile to LDS: phi/rounding/decay for q and k, transposes for k~ and v.
template <typename T, int HD, int TC, int B0, int NB, bool STATE_ONLY>
__device__ __forceinline__ void stage_tile(const uint4 (&raw)[NB * HD / 32], T* sm, int tlen,
                                           float lg, int tid) {
  using LD = Lds<T, HD, TC>;
  constexpr int E = Vec<T>::N;
  constexpr int GPR = HD / E;
  constexpr int NL = NB * HD / 32;
  T* sKt = sm + (STATE_ONLY ? LD::stKt : LD::oKt);
  T* sVt = sm + (STATE_ONLY ? LD::stVt : LD::oVt);
#pragma unroll
  for (int it = 0; it < NL; ++it) {
    const int idx = tid + kThreads * it;
    const int blk = B0 + (kThreads * it) / (TC * GPR);
    const int rem = idx % (TC * GPR);
    const int i = rem / GPR, cg = rem % GPR;
    const bool ok = i < tlen;
    if (blk == 0) {  // q: phi(q) and phi(q)*gamma^i, row-major
      float f[E], fd[E];
      unpack16<T>(raw[it], f);
      const float qd = expf((float)i * lg);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        f[e] = ok ? rnd<T>(phi_f(f[e])) : 0.f;
        fd[e] = f[e] * qd;
      }
      store16<T>(sm + LD::oQ + i * LD::PR + cg * E, f);
      store16<T>(sm + LD::oQd + i * LD::PR + cg * E, fd);
    } else if (blk == 1) {  // k: phi(k) row-major, (phi(k)*gamma^(tlen-1-i))^T
      float f[E];
      unpack16<T>(raw[it], f);
      const float kd = ok ? expf((float)(tlen - 1 - i) * lg) : 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) f[e] = ok ? rnd<T>(phi_f(f[e])) : 0.f;
      if (!STATE_ONLY) store16<T>(sm + LD::oK + i * LD::PR + cg * E, f);
#pragma unroll
      for (int e = 0; e < E; ++e) sKt[(cg * E + e) * LD::PT + i] = from_f<T>(f[e] * kd);
    } else if (blk == 2) {  // v^T
#pragma unroll
      for (int e = 0; e < E; ++e) sVt[(cg * E + e) * LD::PT + i] = raw_elem<T>(raw[it], e);
    } else {  // gate, copied as stored
      *reinterpret_cast<uint4*>(sm + LD::oG + i * LD::PR + cg * E) = raw[it];
    }
  }
}

template <typename T, int HD, int TC, bool HAS_W>
__global__ __launch_bounds__(kThreads) void slot_gate_kernel(
    const T* __restrict__ projs, int64_t prs, int q_col, int dm, int L, int C, int cshift,
    const T* __restrict__ gamma, const T* __restrict__ gn_w, const T* __restrict__ gn_b,
    float gn_eps, const float* __restrict__ Ain, int seg_tiles, int nseg, T* __restrict__ out,
    int64_t ors, int out_col, float* __restrict__ S_final) {
  using LD = Lds<T, HD, TC>;
  static_assert(LD::total * sizeof(T) + 2 * HD * sizeof(float) <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(16))) T sm[LD::total];
  __shared__ float sgw[HD], sgb[HD];
  constexpr int NVT = HD / 16;  // 16-wide tiles across the head dim
  constexpr int NKS = HD / 32;  // K=32 steps across the head dim
  constexpr int NJS = TC / 32;  // K=32 steps across the tile rows
  constexpr int NIT = TC / 16;  // 16-row query tiles
  constexpr int OWN = (NVT + kWaves - 1) / kWaves;
  constexpr int NL = HD / 8;

  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int l16 = lane & 15, kg = lane >> 4;
  const int seg = blockIdx.x, h = blockIdx.y, b = blockIdx.z, H = gridDim.y;
  const float lg = logf(to_f<T>(gamma[h]));
  const int64_t rowbase = (int64_t)b * L;
  const int p_begin = seg * seg_tiles * TC;
  const int p_end = min(L, p_begin + seg_tiles * TC);
  const int colbase = q_col + h * HD;

  if (tid < HD) {
    sgw[tid] = to_f<T>(gn_w[h * HD + tid]);
    sgb[tid] = to_f<T>(gn_b[h * HD + tid]);
  }

  // Carried states: this wave owns dv tiles vt = w + 4*ov; lane holds S[dk][dv] for
  // dk = 16*mt + 4*kg + r, dv = 16*vt + l16.
  f32x4_t stA[OWN][NVT];
  f32x4_t stW[HAS_W ? OWN : 1][HAS_W ? NVT : 1];
  const float* ain = Ain + (((int64_t)b * H + h) * nseg + seg) * HD * HD;
#pragma unroll
  for (int ov = 0; ov < OWN; ++ov) {
    const int vt = w + kWaves * ov;
#pragma unroll
    for (int mt = 0; mt < NVT; ++mt) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        stA[ov][mt][r] = vt < NVT ? ain[(mt * 16 + kg * 4 + r) * HD + vt * 16 + l16] : 0.f;
      if constexpr (HAS_W) stW[ov][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  }
  // S_eff for the first tile (segment starts on a chunk boundary): A.
#pragma unroll
  for (int ov = 0; ov < OWN; ++ov) {
    const int vt = w + kWaves * ov;
    if (vt < NVT) {
#pragma unroll
      for (int mt = 0; mt < NVT; ++mt) {
        float v[4] = {stA[ov][mt][0], stA[ov][mt][1], stA[ov][mt][2], stA[ov][mt][3]};
        store4<T>(sm + LD::oS0 + (vt * 16 + l16) * LD::PR + mt * 16 + kg * 4, v);
      }
    }
  }

  uint4 raw[NL];
  load_tile<T, HD, TC, 0, 4>(raw, projs, prs, rowbase, colbase, dm, p_begin, L, tid);
  int cur = 0;
  for (int p = p_begin; p < p_end; p += TC) {
    const int tlen = min(TC, L - p);
    __syncthreads();
    stage_tile<T, HD, TC, 0, 4, false>(raw, sm, tlen, lg, tid);
    if (p + TC < p_end) load_tile<T, HD, TC, 0, 4>(raw, projs, prs, rowbase, colbase, dm, p + TC, L, tid);
    __syncthreads();
    const T* sS = sm + (cur ? LD::oS1 : LD::oS0);

    // ---- outputs for query rows 16*w .. 16*w+15
    if (w < NIT) {
      const int it = w;
      const int iq = it * 16 + l16;
      f32x4_t yacc[NVT];
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt) yacc[vt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      Frag<T> pf[NJS];
#pragma unroll
      for (int t = 0; t < NJS; ++t) {
        if (2 * t > it) continue;
        float pv[8];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int jt = 2 * t + hh;
          f32x4_t s = {0.f, 0.f, 0.f, 0.f};
          if (jt <= it) {
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
              Frag<T> a, bq;
              frag_load8(a, sm + LD::oK + (jt * 16 + l16) * LD::PR + ks * 32 + kg * 8);
              frag_load8(bq, sm + LD::oQ + iq * LD::PR + ks * 32 + kg * 8);
              s = mma(a, bq, s);
            }
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = jt * 16 + kg * 4 + r;
            float v = 0.f;
            if (jt <= it && j <= iq) {
              const int e = iq - j - (((iq >> cshift) != (j >> cshift)) ? 1 : 0);
              v = s[r] * expf((float)e * lg);
            }
            pv[hh * 4 + r] = v;
          }
        }
        frag_from_f32(pf[t], pv);
      }
      // y^T += V^T P^T (causal: only key tiles <= it)
#pragma unroll
      for (int t = 0; t < NJS; ++t) {
        if (2 * t > it) continue;
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) {
          Frag<T> a;
          const T* base = sm + LD::oVt + (vt * 16 + l16) * LD::PT + 32 * t + kg * 4;
          frag_load4x2(a, base, base + 16);
          yacc[vt] = mma(a, pf[t], yacc[vt]);
        }
      }
      // y^T += S_eff^T (phi(q)*gamma^i)^T
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        Frag<T> bq;
        frag_load8(bq, sm + LD::oQd + iq * LD::PR + ks * 32 + kg * 8);
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) {
          Frag<T> a;
          frag_load8(a, sS + (vt * 16 + l16) * LD::PR + ks * 32 + kg * 8);
          yacc[vt] = mma(a, bq, yacc[vt]);
        }
      }
      // GroupNorm over the head's HD values of row iq, then the sigmoid gate.
      float sum = 0.f;
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
#pragma unroll
        for (int r = 0; r < 4; ++r) sum += yacc[vt][r];
      const float mean = quad_group_sum(sum) * (1.0f / HD);
      float sq = 0.f;
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float d = yacc[vt][r] - mean;
          sq += d * d;
        }
      const float rinv = 1.0f / sqrtf(quad_group_sum(sq) * (1.0f / HD) + gn_eps);
      if (iq < tlen) {
        T* orow = out + (rowbase + p + iq) * ors + out_col + h * HD;
        const T* grow = sm + LD::oG + iq * LD::PR;
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) {
          float o[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int dv = vt * 16 + kg * 4 + r;
            const float yn = (yacc[vt][r] - mean) * rinv * sgw[dv] + sgb[dv];
            const float g = to_f<T>(grow[dv]);
            o[r] = yn * (1.0f / (1.0f + expf(-g)));
          }
          store4<T>(orow + vt * 16 + kg * 4, o);
        }
      }
    }

    // ---- state update: (W or A) <- gamma^tlen * (W or A) + K~^T V
    {
      const float gt = expf((float)tlen * lg);
#pragma unroll
      for (int ov = 0; ov < OWN; ++ov) {
        const int vt = w + kWaves * ov;
        if (vt >= NVT) continue;
        Frag<T> bv[NJS];
#pragma unroll
        for (int ks = 0; ks < NJS; ++ks)
          frag_load8(bv[ks], sm + LD::oVt + (vt * 16 + l16) * LD::PT + ks * 32 + kg * 8);
#pragma unroll
        for (int mt = 0; mt < NVT; ++mt) {
          f32x4_t acc;
          if constexpr (HAS_W) acc = stW[ov][mt] * gt;
          else acc = stA[ov][mt] * gt;
#pragma unroll
          for (int ks = 0; ks < NJS; ++ks) {
            Frag<T> a;
            frag_load8(a, sm + LD::oKt + (mt * 16 + l16) * LD::PT + ks * 32 + kg * 8);
            acc = mma(a, bv[ks], acc);
          }
          if constexpr (HAS_W) stW[ov][mt] = acc;
          else stA[ov][mt] = acc;
        }
      }
      if constexpr (HAS_W) {
        if (((p + tlen) % C) == 0) {
          const float gC = expf((float)C * lg);
#pragma unroll
          for (int ov = 0; ov < OWN; ++ov)
#pragma unroll
            for (int mt = 0; mt < NVT; ++mt) {
              stA[ov][mt] = stA[ov][mt] * gC + stW[ov][mt];
              stW[ov][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
        }
      }
    }

    // ---- S_eff^T for the next tile into the other buffer
    if (p + TC < p_end) {
      T* sSn = sm + (cur ? LD::oS0 : LD::oS1);
      float cA = 1.0f, cW = 0.0f;
      if constexpr (HAS_W) {
        cA = expf((float)((p + TC) % C) * lg);
        cW = expf(lg);
      }
#pragma unroll
      for (int ov = 0; ov < OWN; ++ov) {
        const int vt = w + kWaves * ov;
        if (vt >= NVT) continue;
#pragma unroll
        for (int mt = 0; mt < NVT; ++mt) {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            v[r] = cA * stA[ov][mt][r];
            if constexpr (HAS_W) v[r] += cW * stW[ov][mt][r];
          }
          store4<T>(sSn + (vt * 16 + l16) * LD::PR + mt * 16 + kg * 4, v);
        }
      }
      cur ^= 1;
    }
  }

  if (S_final != nullptr && seg == nseg - 1) {
    float* sf = S_final + ((int64_t)b * H + h) * HD * HD;
#pragma unroll
    for (int ov = 0; ov < OWN; ++ov) {
      const int vt = w + kWaves * ov;
      if (vt >= NVT) continue;
#pragma unroll
      for (int mt = 0; mt < NVT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) sf[(mt * 16 + kg * 4 + r) * HD + vt * 16 + l16] = stA[ov][mt][r];
    }
  }
}

// Per (segment, head, batch): U_s = sum_{j in segment} gamma^(end-1-j) k~_j^T v_j.
template <typename T, int HD, int TC>
__global__ __launch_bounds__(kThreads) void slot_state_kernel(const T* __restrict__ projs,
                                                              int64_t prs, int q_col, int dm,
                                                              int L, const T* __restrict__ gamma,
                                                              int seg_tiles, int nseg,
                                                              float* __restrict__ U) {
  using LD = Lds<T, HD, TC>;
  __shared__ __attribute__((aligned(16))) T sm[LD::stTotal];
  constexpr int NVT = HD / 16;
  constexpr int NJS = TC / 32;
  constexpr int OWN = (NVT + kWaves - 1) / kWaves;
  constexpr int NL = 2 * HD / 32;

  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int l16 = lane & 15, kg = lane >> 4;
  const int seg = blockIdx.x, h = blockIdx.y, b = blockIdx.z, H = gridDim.y;
  const float lg = logf(to_f<T>(gamma[h]));
  const int64_t rowbase = (int64_t)b * L;
  const int p_begin = seg * seg_tiles * TC;
  const int p_end = min(L, p_begin + seg_tiles * TC);
  const int colbase = q_col + h * HD;

  f32x4_t st[OWN][NVT];
#pragma unroll
  for (int ov = 0; ov < OWN; ++ov)
#pragma unroll
    for (int mt = 0; mt < NVT; ++mt) st[ov][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  uint4 raw[NL];
  load_tile<T, HD, TC, 1, 2>(raw, projs, prs, rowbase, colbase, dm, p_begin, L, tid);
  for (int p = p_begin; p < p_end; p += TC) {
    const int tlen = min(TC, L - p);
    __syncthreads();
    stage_tile<T, HD, TC, 1, 2, true>(raw, sm, tlen, lg, tid);
    if (p + TC < p_end) load_tile<T, HD, TC, 1, 2>(raw, projs, prs, rowbase, colbase, dm, p + TC, L, tid);
    __syncthreads();
    const float gt = expf((float)tlen * lg);
#pragma unroll
    for (int ov = 0; ov < OWN; ++ov) {
      const int vt = w + kWaves * ov;
      if (vt >= NVT) continue;
      Frag<T> bv[NJS];
#pragma unroll
      for (int ks = 0; ks < NJS; ++ks)
        frag_load8(bv[ks], sm + LD::stVt + (vt * 16 + l16) * LD::PT + ks * 32 + kg * 8);
#pragma unroll
      for (int mt = 0; mt < NVT; ++mt) {
        f32x4_t acc = st[ov][mt] * gt;
#pragma unroll
        for (int ks = 0; ks < NJS; ++ks) {
          Frag<T> a;
          frag_load8(a, sm + LD::stKt + (mt * 16 + l16) * LD::PT + ks * 32 + kg * 8);
          acc = mma(a, bv[ks], acc);
        }
        st[ov][mt] = acc;
      }
    }
  }
  float* u = U + (((int64_t)b * H + h) * nseg + seg) * HD * HD;
#pragma unroll
  for (int ov = 0; ov < OWN; ++ov) {
    const int vt = w + kWaves * ov;
    if (vt >= NVT) continue;
#pragma unroll
    for (int mt = 0; mt < NVT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) u[(mt * 16 + kg * 4 + r) * HD + vt * 16 + l16] = st[ov][mt][r];
  }
}

// Per (element, head, batch): Ain[s] = state at the start of segment s.
template <typename T>
__global__ __launch_bounds__(kThreads) void slot_scan_kernel(const float* __restrict__ U,
                                                             const float* __restrict__ S0,
                                                             float* __restrict__ Ain,
                                                             const T* __restrict__ gamma, int HD2,
                                                             int nseg, int seg_len) {
  const int e = blockIdx.x * kThreads + threadIdx.x;
  const int h = blockIdx.y, b = blockIdx.z, H = gridDim.y;
  if (e >= HD2) return;
  const float gs = expf((float)seg_len * logf(to_f<T>(gamma[h])));
  const int64_t bh = (int64_t)b * H + h;
  float a = S0 ? S0[bh * HD2 + e] : 0.f;
  const int64_t base = bh * nseg * HD2 + e;
  for (int s = 0; s < nseg; ++s) {
    Ain[base + (int64_t)s * HD2] = a;
    if (s + 1 < nseg) a = a * gs + U[base + (int64_t)s * HD2];
  }
}

struct SlotPlan {
  int HD, TC, seg_tiles, nseg, cshift;
  bool has_w;
};

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  if (!v || !*v) return dflt;
  const int x = atoi(v);
  return x > 0 ? x : dflt;
}

int slot_plan(int64_t B, int64_t L, int64_t dm, int64_t H, int64_t C, int dtype, SlotPlan* pl) {
  if (dtype != HDCM_F32 && dtype != HDCM_BF16) return HDCM_EUNSUPPORTED;
  if (B < 0 || L < 0 || dm <= 0 || H <= 0 || C <= 0 || dm % H) return HDCM_EINVAL;
  const int64_t HD = dm / H;
  if (HD != 32 && HD != 64 && HD != 96) return HDCM_EUNSUPPORTED;
  const int TC = dtype == HDCM_BF16 ? 64 : 32;
  if (L % C) return HDCM_EINVAL;
  int cshift = 31;
  if (C < TC) {
    if (TC % C) return HDCM_EUNSUPPORTED;
    cshift = 0;
    while ((1 << cshift) < C) ++cshift;
  } else if (C % TC) {
    return HDCM_EUNSUPPORTED;
  }
  if (B > 65535 || H > 65535) return HDCM_EUNSUPPORTED;
  const int64_t tiles = (L + TC - 1) / TC;
  const int64_t unit = C > TC ? C / TC : 1;
  int64_t st = env_int("HDCM_SLOT_SEG_TILES", 0);
  if (st == 0) {
    const int64_t bh = B * H > 0 ? B * H : 1;
    const int64_t want = (kTargetWorkgroups + bh - 1) / bh;
    st = (tiles + want - 1) / want;
    if (st < kMinSegTiles) st = kMinSegTiles;
  }
  st = (st + unit - 1) / unit * unit;
  const int64_t cap = (tiles + unit - 1) / unit * unit;
  if (st > cap) st = cap;
  if (st < 1) st = 1;
  pl->HD = (int)HD;
  pl->TC = TC;
  pl->seg_tiles = (int)st;
  pl->nseg = (int)((tiles + st - 1) / st);
  if (pl->nseg < 1) pl->nseg = 1;
  pl->cshift = cshift;
  pl->has_w = C > TC;
  if (pl->nseg > 65535 || L > ((int64_t)1 << 30)) return HDCM_EUNSUPPORTED;
  return HDCM_OK;
}

size_t slot_ws_bytes(int64_t B, int64_t H, const SlotPlan& pl) {
  return (size_t)2 * B * H * pl.nseg * pl.HD * pl.HD * sizeof(float);
}

template <typename T, int HD>
int launch_state(const void* projs, int64_t prs, int64_t q_col, const void* gamma,
                 const float* S0, void* ws, int64_t B, int64_t L, int64_t dm, int64_t H,
                 const SlotPlan& pl, hipStream_t s) {
  constexpr int TC = TileOf<T>::value;
  float* U = (float*)ws;
  float* Ain = U + (size_t)B * H * pl.nseg * HD * HD;
  if (pl.nseg > 1) {
    hipLaunchKernelGGL((slot_state_kernel<T, HD, TC>), dim3(pl.nseg - 1, (unsigned)H, (unsigned)B),
                       dim3(kThreads), 0, s, (const T*)projs, prs, (int)q_col, (int)dm, (int)L,
                       (const T*)gamma, pl.seg_tiles, pl.nseg, U);
    const int st = hdcm_launch_status();
    if (st) return st;
  }
  hipLaunchKernelGGL((slot_scan_kernel<T>), dim3((HD * HD + kThreads - 1) / kThreads, (unsigned)H, (unsigned)B),
                     dim3(kThreads), 0, s, U, S0, Ain, (const T*)gamma, HD * HD, pl.nseg,
                     pl.seg_tiles * TC);
  return hdcm_launch_status();
}

template <typename T, int HD>
int launch_gate(const void* projs, int64_t prs, int64_t q_col, const void* gamma,
                const void* gn_w, const void* gn_b, float gn_eps, const void* ws, void* out,
                int64_t ors, int64_t out_col, float* S_final, int64_t B, int64_t L, int64_t dm,
                int64_t H, int64_t C, const SlotPlan& pl, hipStream_t s) {
  constexpr int TC = TileOf<T>::value;
  const float* Ain = (const float*)ws + (size_t)B * H * pl.nseg * HD * HD;
  dim3 grid(pl.nseg, (unsigned)H, (unsigned)B);
  if (pl.has_w)
    hipLaunchKernelGGL((slot_gate_kernel<T, HD, TC, true>), grid, dim3(kThreads), 0, s,
                       (const T*)projs, prs, (int)q_col, (int)dm, (int)L, (int)C, pl.cshift,
                       (const T*)gamma, (const T*)gn_w, (const T*)gn_b, gn_eps, Ain, pl.seg_tiles,
                       pl.nseg, (T*)out, ors, (int)out_col, S_final);
  else
    hipLaunchKernelGGL((slot_gate_kernel<T, HD, TC, false>), grid, dim3(kThreads), 0, s,
                       (const T*)projs, prs, (int)q_col, (int)dm, (int)L, (int)C, pl.cshift,
                       (const T*)gamma, (const T*)gn_w, (const T*)gn_b, gn_eps, Ain, pl.seg_tiles,
                       pl.nseg, (T*)out, ors, (int)out_col, S_final);
  return hdcm_launch_status();
}

int check_projs(const void* projs, int64_t prs, int64_t q_col, int64_t dm, int dtype) {
  const int E = 16 / hdcm_elt_size(dtype);
  if (!projs) return HDCM_EINVAL;
  if (q_col < 0 || prs < q_col + 4 * dm) return HDCM_EINVAL;
  if (!hdcm_aligned16(projs) || prs % E || q_col % E || dm % E) return HDCM_EALIGN;
  return HDCM_OK;
}

}  // namespace

extern "C" size_t hdcm_slot_workspace_bytes(int64_t B, int64_t L, int64_t dm, int64_t H, int64_t C,
                                            int dtype) {
  SlotPlan pl;
  if (slot_plan(B, L, dm, H, C, dtype, &pl) != HDCM_OK) return 0;
  return slot_ws_bytes(B, H, pl);
}

extern "C" int hdcm_slot_state_fwd(const void* projs, int64_t proj_row_stride, int64_t q_col,
                                   const void* gamma, const float* S0, void* ws, size_t ws_bytes,
                                   int64_t B, int64_t L, int64_t dm, int64_t H, int64_t C,
                                   int dtype, void* stream) {
  SlotPlan pl;
  int st = slot_plan(B, L, dm, H, C, dtype, &pl);
  if (st) return st;
  st = check_projs(projs, proj_row_stride, q_col, dm, dtype);
  if (st) return st;
  HDCM_CHECK_ARG(gamma != nullptr, HDCM_EINVAL);
  if (B == 0 || L == 0) return HDCM_OK;
  HDCM_CHECK_ARG(ws != nullptr && ws_bytes >= slot_ws_bytes(B, H, pl), HDCM_EWORKSPACE);
  HDCM_CHECK_ARG(((uintptr_t)ws & 15u) == 0, HDCM_EALIGN);
  hipStream_t s = (hipStream_t)stream;
#define HDCM_STATE_CASE(TT, HDV)                                                                  \
  if (pl.HD == HDV)                                                                              \
    return launch_state<TT, HDV>(projs, proj_row_stride, q_col, gamma, S0, ws, B, L, dm, H, pl, s);
  if (dtype == HDCM_BF16) {
    HDCM_STATE_CASE(bf16_t, 32)
    HDCM_STATE_CASE(bf16_t, 64)
    HDCM_STATE_CASE(bf16_t, 96)
  } else {
    HDCM_STATE_CASE(float, 32)
    HDCM_STATE_CASE(float, 64)
    HDCM_STATE_CASE(float, 96)
  }
#undef HDCM_STATE_CASE
  return HDCM_EUNSUPPORTED;
}

extern "C" int hdcm_slot_gate_fwd(const void* projs, int64_t proj_row_stride, int64_t q_col,
                                  const void* gamma, const void* gn_w, const void* gn_b,
                                  float gn_eps, const void* ws, size_t ws_bytes, void* out,
                                  int64_t out_row_stride, int64_t out_col, float* S_final,
                                  int64_t B, int64_t L, int64_t dm, int64_t H, int64_t C,
                                  int dtype, void* stream) {
  SlotPlan pl;
  int st = slot_plan(B, L, dm, H, C, dtype, &pl);
  if (st) return st;
  st = check_projs(projs, proj_row_stride, q_col, dm, dtype);
  if (st) return st;
  HDCM_CHECK_ARG(gamma && gn_w && gn_b && out, HDCM_EINVAL);
  const int esz = hdcm_elt_size(dtype);
  HDCM_CHECK_ARG(out_col >= 0 && out_row_stride >= out_col + dm, HDCM_EINVAL);
  // Output runs of 4 elements must be naturally aligned (8 bytes bf16, 16 bytes fp32).
  HDCM_CHECK_ARG(((uintptr_t)out % (4 * esz)) == 0 && out_col % 4 == 0 && out_row_stride % 4 == 0,
                 HDCM_EALIGN);
  if (B == 0 || L == 0) return HDCM_OK;
  HDCM_CHECK_ARG(ws != nullptr && ws_bytes >= slot_ws_bytes(B, H, pl), HDCM_EWORKSPACE);
  HDCM_CHECK_ARG(((uintptr_t)ws & 15u) == 0, HDCM_EALIGN);
  hipStream_t s = (hipStream_t)stream;
#define HDCM_GATE_CASE(TT, HDV)                                                                 \
  if (pl.HD == HDV)                                                                            \
    return launch_gate<TT, HDV>(projs, proj_row_stride, q_col, gamma, gn_w, gn_b, gn_eps, ws, \
                                out, out_row_stride, out_col, S_final, B, L, dm, H, C, pl, s);
  if (dtype == HDCM_BF16) {
    HDCM_GATE_CASE(bf16_t, 32)
    HDCM_GATE_CASE(bf16_t, 64)
    HDCM_GATE_CASE(bf16_t, 96)
  } else {
    HDCM_GATE_CASE(float, 32)
    HDCM_GATE_CASE(float, 64)
    HDCM_GATE_CASE(float, 96)
  }
#undef HDCM_GATE_CASE
  return HDCM_EUNSUPPORTED;
}
