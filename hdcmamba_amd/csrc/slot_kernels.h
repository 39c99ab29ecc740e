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
// factor gamma^-1 appears inside the tile's score matrix instead.  Any other C is walked in
// chunk-confined tiles: each chunk is covered by ceil(C/TC) tiles of up to TC rows (the last
// one shorter), so no tile straddles a chunk boundary (the rows past a short tile are zero
// in LDS) and the W/A split above applies unchanged.
//
// Head dims: any multiple of 16 up to 128.  The contractions over the head dim run in K=32
// steps, so for hd not a multiple of 32 the phi(q), phi(k) and S_eff^T tiles carry zero
// columns up to the next multiple of 32 (written once per workgroup); contractions over
// tokens and the value columns use the hd/16 16-wide tiles as they are.
//
// Parallelism: the sequence is cut into segments of whole tiles that start on chunk
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
// is shared through an LDS tile written while the next row tile is staged.
#pragma once

#include <stdlib.h>

#include <type_traits>

#include "hdcm_common.h"

using namespace hdcm;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
// Segments are sized for about two workgroups per CU (512 on 256 CUs).  At B=1, L=32768,
// 16 heads the measured forward prefers 16 tiles per segment (512 workgroups) to 8 (1024,
// 1.3 rounds of the gate pass at 3 workgroups per CU) and to 4-13 or 22.
constexpr int kTargetWorkgroups = 512;
constexpr int kGateWavesPerEU = 3;  // register budget: 3 waves per SIMD (3 workgroups per CU)
constexpr int kMinSegTiles = 4;

template <typename T>
struct TileOf {
  static constexpr int value = sizeof(T) == 2 ? 64 : 32;
};

// LDS tiles of one row tile.  phi(q), phi(k) and S_eff^T feed the MFMAs through 16-byte
// reads along the head dim; they are row-major with a pitch of HD plus one 16-byte chunk,
// which puts the reads of 16 consecutive rows on distinct banks.  k~ = phi(k)*decay and v
// feed P.V and the state update along the token dim.  For bf16 they stay row-major
// (pitch HD+16, 16-byte stores) and are read with ds_read_tr16_b64, which hands each lane
// 4 consecutive tokens of one column; for fp32 they are stored transposed, [HD][TC].
template <typename T, int HD, int TC>
struct Lds {
  static constexpr bool TR = sizeof(T) == 2;
  static constexpr int E = 16 / sizeof(T);
  static constexpr int HDK = (HD + 31) / 32 * 32;  // contraction width over the head dim
  static constexpr int PQ = HDK + E;
  static constexpr int PV = TR ? HD + 16 : TC + E;
  static constexpr int tileQ = TC * PQ;
  static constexpr int tileV = TR ? TC * PV : HD * PV;
  static constexpr int oQ = 0;             // phi(q)
  static constexpr int oK = oQ + tileQ;    // phi(k)
  static constexpr int oKd = oK + tileQ;   // k~ = phi(k) * gamma^(tlen-1-i)
  static constexpr int oV = oKd + tileV;   // v
  static constexpr int oS = oV + tileV;    // S_eff^T [HD][HDK]
  static constexpr int total = oS + HD * PQ;
  // the state pre-pass uses only k~ and v
  static constexpr int stKd = 0;
  static constexpr int stV = tileV;
  static constexpr int stTotal = 2 * tileV;
};

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));

// Transpose read: within each 16-lane group, lane c supplies the address of 4 consecutive
// 16-bit elements; lane x receives element x%4 of the chunks supplied by lanes x/4,
// x/4+4, x/4+8 and x/4+12.
__device__ __forceinline__ bf16x4_t lds_tr16(const bf16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4_t*)p);
}

// Head-dim fragment: columns col..col+7 of `row` of a PQ-pitched tile.
template <typename T, int HD, int TC>
__device__ __forceinline__ void frag_rows8(Frag<T>& f, const T* tile, int row, int col) {
  frag_load8(f, tile + row * Lds<T, HD, TC>::PQ + col);
}

// Token-dim fragment of k~ or v: lane (x = lane%16, g = lane/16) receives, for head-dim
// column d0 + x, tokens j0 + 4g + s in slots s = 0..3 and j0 + 16 + 4g + s - 4 in slots
// 4..7 -- the slot order of the score fragments, used for every token contraction.
template <typename T, int HD, int TC>
__device__ __forceinline__ void frag_tok(Frag<T>& f, const T* tile, int d0, int j0, int lane) {
  using LD = Lds<T, HD, TC>;
  const int x = lane & 15, g = lane >> 4;
  if constexpr (LD::TR) {
    // lane c of the group points at token j0 + 4g + c/4, columns d0 + 4*(c%4) .. +3
    const T* p = tile + (j0 + 4 * g + (x >> 2)) * LD::PV + d0 + 4 * (x & 3);
    const bf16x4_t lo = lds_tr16(p);
    const bf16x4_t hi = lds_tr16(p + 16 * LD::PV);
    f.v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  } else {
    const T* p = tile + (d0 + x) * LD::PV + j0 + 4 * g;
    frag_load4x2(f, p, p + 16);
  }
}


template <typename T>
__device__ __forceinline__ void store4(T* p, const float* v);
template <>
__device__ __forceinline__ void store4<float>(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
template <>
__device__ __forceinline__ void store4<bf16_t>(bf16_t* p, const float* v) {
  *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
}

// 4 consecutive elements from global memory as fp32.
template <typename T>
__device__ __forceinline__ void load4(const T* p, float* v);
template <>
__device__ __forceinline__ void load4<float>(const float* p, float* v) {
  const float4 u = *reinterpret_cast<const float4*>(p);
  v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
}
template <>
__device__ __forceinline__ void load4<bf16_t>(const bf16_t* p, float* v) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  v[0] = __uint_as_float(u.x << 16); v[1] = __uint_as_float(u.x & 0xffff0000u);
  v[2] = __uint_as_float(u.y << 16); v[3] = __uint_as_float(u.y & 0xffff0000u);
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

// Scale the 8 slots of a fragment by c, rounding to the operand type.
__device__ __forceinline__ Frag<bf16_t> frag_scale(const Frag<bf16_t>& f, float c) {
  float x[8];
  unpack_bf16x8(f.v, x);
#pragma unroll
  for (int s = 0; s < 8; ++s) x[s] *= c;
  Frag<bf16_t> o;
  o.v = pack_bf16x8(x);
  return o;
}
__device__ __forceinline__ Frag<float> frag_scale(const Frag<float>& f, float c) {
  Frag<float> o;
#pragma unroll
  for (int s = 0; s < 8; ++s) o.v[s] = f.v[s] * c;
  return o;
}

// Tile loader.  The tile's q, k, v (blocks 0,1,2) or only k, v (B0=1, NB=2) are split
// into 16-byte groups, GPT = TC*GPR of them per block; iteration it covers block
// B0 + it/IPB, group idx = tid + 256*(it%IPB) (row idx/GPR, column group idx%GPR), so the
// block of each iteration is uniform and rows advance by whole tiles between calls.  When
// GPT is not a multiple of 256 the threads past it in a block's last iteration are idle:
// they load row 0, column group 0 of the block (in bounds) and stage nothing.  Block B0+k
// starts boff[k] columns after the tile base (the q, k, v column blocks of one row buffer).
// The row stride may be negative (a sequence walked backwards from its last row).
template <typename T, int HD, int TC, int B0, int NB>
struct TileLoader {
  static constexpr int E = Vec<T>::N;
  static constexpr int GPR = HD / E;
  static constexpr int GPT = TC * GPR;                           // groups per block
  static constexpr int IPB = (GPT + kThreads - 1) / kThreads;    // iterations per block
  static constexpr int NL = NB * IPB;
  static constexpr bool EXACT = GPT % kThreads == 0;
  static constexpr bool SCALAR = EXACT && (kThreads % GPR) == 0;  // row step per iteration is uniform
  static_assert(HD % E == 0, "head dim in 16-byte groups");
  // With SCALAR, iteration it reads row tid/GPR + (it % IPB) * (kThreads/GPR) of block
  // B0 + it/IPB at column group tid%GPR: one per-thread offset plus uniform strides.
  int64_t base;
  int row0;
  int64_t prs;
  int boff[NB];
  int64_t off[SCALAR ? 1 : NL];
  int row[SCALAR ? 1 : NL];
  __device__ __forceinline__ static bool valid(int it, int tid) {
    return EXACT || tid + kThreads * (it % IPB) < GPT;
  }
  __device__ __forceinline__ TileLoader(int64_t prs_, const int (&boffs)[NB], int tid) : prs(prs_) {
#pragma unroll
    for (int k = 0; k < NB; ++k) boff[k] = boffs[k];
    row0 = tid / GPR;
    base = (int64_t)row0 * prs + (tid % GPR) * E;
    if constexpr (!SCALAR) {
#pragma unroll
      for (int it = 0; it < NL; ++it) {
        const int idx = tid + kThreads * (it % IPB);
        const int blk = it / IPB;
        if (valid(it, tid)) {
          row[it] = idx / GPR;
          off[it] = (int64_t)row[it] * prs + boff[blk] + (idx % GPR) * E;
        } else {
          row[it] = 0;
          off[it] = boff[blk];
        }
      }
    }
  }
  __device__ __forceinline__ int row_of(int it) const {
    if constexpr (SCALAR) return row0 + (it % IPB) * (kThreads / GPR);
    else return row[it];
  }
  __device__ __forceinline__ int64_t off_of(int it) const {
    if constexpr (SCALAR)
      return base + (int64_t)((it % IPB) * (kThreads / GPR)) * prs + boff[it / IPB];
    else return off[it];
  }
  // Always NL loads, whatever tlen (>= 1): a fixed count per tile keeps the compiler's
  // memory-counter waits exact instead of draining every outstanding load.  Rows past the
  // tile read row 0 of the tile and are zeroed when staged.
  __device__ __forceinline__ void load(uint4 (&raw)[NL], const T* tile_base, int tlen) const {
#pragma unroll
    for (int it = 0; it < NL; ++it) {
      const int r = row_of(it);
      const int64_t off = off_of(it);
      raw[it] = ldg16(tile_base + (r < tlen ? off : off - (int64_t)r * prs));
    }
  }
};

// Write a loaded tile to LDS.  q: phi(q) row-major.  k: phi(k) row-major (unless
// STATE_ONLY) and (phi(k)*gamma^(tlen-1-i))^T.  v: v^T.  Rows >= tlen are zero.  Without
// PHI the feature map is the identity (q and k staged as they are).
template <typename T, int HD, int TC, int B0, int NB, bool STATE_ONLY, bool PHI, bool FULL>
__device__ __forceinline__ void stage_tile_impl(const uint4 (&raw)[TileLoader<T, HD, TC, B0, NB>::NL], T* sm,
                                                int tlen, float lg2, int tid) {
  using LD = Lds<T, HD, TC>;
  using TL = TileLoader<T, HD, TC, B0, NB>;
  constexpr int E = TL::E, GPR = TL::GPR;
  T* sKd = sm + (STATE_ONLY ? LD::stKd : LD::oKd);
  T* sV = sm + (STATE_ONLY ? LD::stV : LD::oV);
#pragma unroll
  for (int it = 0; it < TL::NL; ++it) {
    if (!TL::valid(it, tid)) continue;
    const int idx = tid + kThreads * (it % TL::IPB);
    const int blk = B0 + it / TL::IPB;
    const int i = idx / GPR, cg = idx % GPR;
    const bool ok = FULL || i < tlen;
    if (blk == 0) {  // phi(q), row-major
      float f[E];
      unpack16<T>(raw[it], f);
#pragma unroll
      for (int e = 0; e < E; ++e) f[e] = ok ? (PHI ? phi_f(f[e]) : f[e]) : 0.f;
      store16<T>(sm + LD::oQ + i * LD::PQ + cg * E, f);
    } else if (blk == 1) {  // phi(k) row-major; k~ = round(phi(k)) * gamma^(tlen-1-i)
      float f[E], kdv[E];
      unpack16<T>(raw[it], f);
      const float kd = ok ? fexp2((float)(tlen - 1 - i) * lg2) : 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) f[e] = ok ? (PHI ? phi_f(f[e]) : f[e]) : 0.f;
      if constexpr (sizeof(T) == 2) {
        // round phi(k) once, in pairs; the rounded words are stored as they are
        const bf16x8_t pk = pack_bf16x8(f);
        if (!STATE_ONLY) *reinterpret_cast<bf16x8_t*>(sm + LD::oK + i * LD::PQ + cg * E) = pk;
        unpack_bf16x8(pk, f);
      } else {
        if (!STATE_ONLY) store16<T>(sm + LD::oK + i * LD::PQ + cg * E, f);
      }
#pragma unroll
      for (int e = 0; e < E; ++e) kdv[e] = f[e] * kd;
      if constexpr (LD::TR) {
        store16<T>(sKd + i * LD::PV + cg * E, kdv);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) sKd[(cg * E + e) * LD::PV + i] = from_f<T>(kdv[e]);
      }
    } else {  // v as stored
      const uint4 vv = ok ? raw[it] : make_uint4(0, 0, 0, 0);
      if constexpr (LD::TR) {
        *reinterpret_cast<uint4*>(sV + i * LD::PV + cg * E) = vv;
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) sV[(cg * E + e) * LD::PV + i] = raw_elem<T>(vv, e);
      }
    }
  }
}

template <typename T, int HD, int TC, int B0, int NB, bool STATE_ONLY, bool PHI>
__device__ __forceinline__ void stage_tile(const uint4 (&raw)[TileLoader<T, HD, TC, B0, NB>::NL], T* sm,
                                           int tlen, float lg2, int tid) {
  if (tlen == TC)
    stage_tile_impl<T, HD, TC, B0, NB, STATE_ONLY, PHI, true>(raw, sm, tlen, lg2, tid);
  else
    stage_tile_impl<T, HD, TC, B0, NB, STATE_ONLY, PHI, false>(raw, sm, tlen, lg2, tid);
}

// Zero the contraction padding of the row-major tiles (columns HD .. HDK-1 of phi(q), phi(k)
// and S_eff^T), which staging never writes: once per workgroup, before the first barrier.
template <typename T, int HD, int TC>
__device__ __forceinline__ void zero_contraction_pad(T* sm, int tid) {
  using LD = Lds<T, HD, TC>;
  constexpr int PAD = LD::HDK - HD;
  if constexpr (PAD > 0) {
    constexpr int ROWS = 2 * TC + HD;  // phi(q) and phi(k) rows, then S_eff^T rows
    for (int k = tid; k < ROWS * PAD; k += kThreads) {
      const int r = k / PAD, c = HD + k % PAD;
      T* t = r < TC ? sm + LD::oQ + r * LD::PQ : r < 2 * TC ? sm + LD::oK + (r - TC) * LD::PQ
                                                           : sm + LD::oS + (r - 2 * TC) * LD::PQ;
      t[c] = T();
    }
  }
}

// PHI: feature map phi on q and k (else the identity).  EPI: GroupNorm + sigmoid gate
// epilogue (else y itself is stored).  CHAIN (without EPI): each stored value is multiplied by
// phi'(z) = 1 (z > 0) else exp(z), z read from zb at the output's own row and column (zb has
// the output's column layout, row stride zrs) — the feature map's chain rule of a gradient
// pass.  k, v and the gate start k_off, v_off, g_off columns after q in each row.  CONF: tiles
// are chunk-confined (a C that neither divides TC nor is a multiple of it); otherwise every
// tile but a segment's last has TC rows, and the loop steps by the constant TC.
template <typename T, int HD, int TC, bool HAS_W, bool PAIRS, bool PHI, bool EPI, bool CHAIN = false,
          bool CONF = false>
__global__ __launch_bounds__(kThreads, HD > 64 ? 1 : (HAS_W ? 2 : kGateWavesPerEU)) void slot_gate_kernel(
    const T* __restrict__ projs, int64_t prs, int q_col, int k_off, int v_off, int g_off, int L, int C, int cshift,
    const T* __restrict__ gamma, const T* __restrict__ gn_w, const T* __restrict__ gn_b,
    float gn_eps, const float* __restrict__ Ain, int seg_rows, int nseg, T* __restrict__ out,
    int64_t ors, int out_col, float* __restrict__ S_final, float* __restrict__ row_stats, int64_t stats_ps,
    const T* __restrict__ zb = nullptr, int64_t zrs = 0) {
  using LD = Lds<T, HD, TC>;
  using TL = TileLoader<T, HD, TC, 0, 3>;
  static_assert(LD::total * sizeof(T) + 2 * HD * sizeof(float) <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(16))) T sm[LD::total];
  __shared__ float sgw[HD], sgb[HD];
  constexpr int NVT = HD / 16;  // 16-wide tiles across the head dim
  constexpr int NKS = LD::HDK / 32;  // K=32 steps across the head dim (zero-padded)
  constexpr int NJS = TC / 32;       // K=32 steps across the tile rows
  constexpr int NIT = TC / 16;       // 16-row query tiles
  constexpr int OWN = (NVT + kWaves - 1) / kWaves;

  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int l16 = lane & 15, kg = lane >> 4;
  const int h = blockIdx.x, seg = blockIdx.y, b = blockIdx.z, H = gridDim.x;
  // gamma and the GroupNorm affine are loaded first and used only after the start state and
  // the first tile have been requested, so no wait comes before those loads
  const T gamma_raw = gamma[h];
  T gnw_raw = T(), gnb_raw = T();
  if constexpr (EPI) {  // every lane loads (a clamped column), so no branch holds a wait
    gnw_raw = gn_w[h * HD + tid % HD];
    gnb_raw = gn_b[h * HD + tid % HD];
  }
  // cshift >= 31: C >= TC or tiles are chunk-confined (CONF), so every pair in a tile shares
  // a chunk; otherwise tiles hold TC/C whole chunks
  const bool one_chunk = cshift >= 31;
  const int64_t rowbase = (int64_t)b * L;
  const int p_begin = seg * seg_rows;
  const int p_end = min(L, p_begin + seg_rows);
  // rows of the tile starting at p (p_end, and with CONF chunk ends, are tile ends)
  auto tile_len = [&](int p) {
    if constexpr (CONF) return min(min(TC, p_end - p), C - p % C);
    else return min(TC, p_end - p);
  };
  const T* colbase = projs + q_col + h * HD;
  // the gate (EPI), or the chain rule's z (CHAIN: same positions as the output)
  const T* gatebase = CHAIN ? zb + out_col + h * HD : colbase + g_off;
  const int64_t grs = CHAIN ? zrs : prs;

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

  const TL loader(prs, {0, k_off, v_off}, tid);
  uint4 raw[TL::NL];
  loader.load(raw, colbase + (rowbase + p_begin) * prs, tile_len(p_begin));

  // Gate values of this lane's output positions (row 16*w + l16 of a tile), kept as
  // stored.  They are loaded one tile ahead, right after the current tile's outputs, so
  // the load overlaps the state update, the next tile's staging and both barriers.  Rows
  // past the tile read the tile's first row (never stored), which keeps the load count
  // fixed and the memory-counter waits exact.
  //   fp32: columns 16*vt + 4*kg .. +3 of every 16-column tile vt (16 bytes each).
  //   bf16 with 16-byte aligned output rows (PAIRS): 16-byte runs in the exchanged layout
  //   of the output stage below: for each pair of tiles, columns
  //   32*pp + 16*(kg&1) + 8*(kg>>1) .. +7.  Otherwise as fp32 (8 bytes each).
  constexpr bool kPairs = PAIRS && sizeof(T) == 2 && NVT % 2 == 0;  // odd tile counts: 8-byte runs
  constexpr int NG = kPairs ? NVT / 2 : NVT;
  const int gcol = kPairs ? 16 * (kg & 1) + 8 * (kg >> 1) : 4 * kg;
  const int gstep = kPairs ? 32 : 16;
  uint4 graw[NG];
  const int giq = (w < NIT ? w : 0) * 16 + l16;
  auto load_gate = [&](int pt) {
    const int tl = tile_len(pt);
    const T* grow = gatebase + (rowbase + pt + (giq < tl ? giq : 0)) * grs + gcol;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if constexpr (kPairs || sizeof(T) == 4) {
        graw[g] = *reinterpret_cast<const uint4*>(grow + g * gstep);
      } else {
        // bf16 without 16-byte runs: the 4 values used (8 bytes), so the last head's read
        // ends at its own last column
        const uint2 v = *reinterpret_cast<const uint2*>(grow + g * gstep);
        graw[g] = make_uint4(v.x, v.y, 0u, 0u);
      }
    }
  };
  if ((EPI || CHAIN) && w < NIT) load_gate(p_begin);

  const float lg2 = log2f(to_f<T>(gamma_raw));
  const float ginv[4] = {1.0f, fexp2(-lg2), fexp2(-2.0f * lg2), fexp2(-3.0f * lg2)};
  if (EPI && tid < HD) {  // read after the loop's first barrier
    sgw[tid] = to_f<T>(gnw_raw);
    sgb[tid] = to_f<T>(gnb_raw);
  }
  zero_contraction_pad<T, HD, TC>(sm, tid);  // ordered before every read by the loop's barriers

  for (int p = p_begin; p < p_end; p += CONF ? tile_len(p) : TC) {
    const int tlen = tile_len(p);
    __syncthreads();
    stage_tile<T, HD, TC, 0, 3, false, PHI>(raw, sm, tlen, lg2, tid);
    // S_eff^T for this tile: gamma*W + gamma^(p-cs)*A (A alone when C divides TC).
    {
      float cA = 1.0f, cW = 0.0f;
      if constexpr (HAS_W) {
        cA = fexp2((float)(p % C) * lg2);
        cW = fexp2(lg2);
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
          store4<T>(sm + LD::oS + (vt * 16 + l16) * LD::PQ + mt * 16 + kg * 4, v);
        }
      }
    }
    {
      // next tile, or this tile again (already in cache) after the last: a fixed load count
      const int pn = p + tlen < p_end ? p + tlen : p;
      loader.load(raw, colbase + (rowbase + pn) * prs, tile_len(pn));
    }
    __syncthreads();

    // ---- outputs for query rows 16*w .. 16*w+15
    if (w < NIT) {
      const int it = w;
      const int iq = it * 16 + l16;
      f32x4_t yacc[NVT];
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt) yacc[vt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      Frag<T> bq[NKS];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) frag_rows8<T, HD, TC>(bq[ks], sm + LD::oQ, iq, ks * 32 + kg * 8);
      // y^T += S_eff^T (phi(q)*gamma^iq)^T
      {
        const float qd = fexp2((float)iq * lg2);
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const Frag<T> bqd = frag_scale(bq[ks], qd);
#pragma unroll
          for (int vt = 0; vt < NVT; ++vt) {
            Frag<T> a;
            frag_rows8<T, HD, TC>(a, sm + LD::oS, vt * 16 + l16, ks * 32 + kg * 8);
            yacc[vt] = mma(a, bqd, yacc[vt]);
          }
        }
      }
      // scores S^T[j][iq] for key tiles j <= it, decayed and masked, as P^T fragments
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
              Frag<T> a;
              frag_rows8<T, HD, TC>(a, sm + LD::oK, jt * 16 + l16, ks * 32 + kg * 8);
              s = mma(a, bq[ks], s);
            }
          }
          if (one_chunk) {
            // gamma^(iq-j) = gamma^(iq-j0) * gamma^-r for the lane's 4 rows j = j0 + r
            const int j0 = jt * 16 + kg * 4;
            const float d0 = fexp2((float)(iq - j0) * lg2);
#pragma unroll
            for (int r = 0; r < 4; ++r)
              pv[hh * 4 + r] = (jt <= it && j0 + r <= iq) ? s[r] * (d0 * ginv[r]) : 0.f;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int j = jt * 16 + kg * 4 + r;
              const int e = iq - j - (((iq >> cshift) != (j >> cshift)) ? 1 : 0);
              pv[hh * 4 + r] = (jt <= it && j <= iq) ? s[r] * fexp2((float)e * lg2) : 0.f;
            }
          }
        }
        Frag<T> pf;
        frag_from_f32(pf, pv);
        // y^T += V^T P^T over the 32 key rows of this step
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) {
          Frag<T> a;
          frag_tok<T, HD, TC>(a, sm + LD::oV, vt * 16, 32 * t, lane);
          yacc[vt] = mma(a, pf, yacc[vt]);
        }
      }
      // GroupNorm over the head's HD values of row iq, then the sigmoid gate (EPI); else y.
      float mean = 0.f, rinv = 1.f;
      if constexpr (EPI) {
        float sum = 0.f;
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt)
#pragma unroll
          for (int r = 0; r < 4; ++r) sum += yacc[vt][r];
        mean = quad_group_sum(sum) * (1.0f / HD);
        float sq = 0.f;
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float d = yacc[vt][r] - mean;
            sq += d * d;
          }
        rinv = rsqrtf(quad_group_sum(sq) * (1.0f / HD) + gn_eps);
      }
      // output value of column vt*16 + 4*kg + r of row iq, given its gate value
      auto out_val = [&](int vt, int r, float gv) -> float {
        if constexpr (EPI) {
          const int dv = vt * 16 + kg * 4 + r;
          const float yn = (yacc[vt][r] - mean) * rinv * sgw[dv] + sgb[dv];
          return yn * frcp(1.0f + fexp(-gv));
        } else {
          return yacc[vt][r];
        }
      };
      // with row_stats (EPI): the sum and sum of squares of the stored (rounded) values of row
      // iq over the head's HD columns, the partial statistics of the row LayerNorm after it
      float st_s = 0.f, st_q = 0.f;
      if constexpr (kPairs) {
        // Tiles vt = 2pp and 2pp+1 leave this lane 4+4 values of row iq; one
        // v_permlane16_swap per packed word trades them between the lane pairs (kg, kg^1) of
        // the same row so that every lane ends with 8 consecutive columns (kg=0: tile 2pp
        // cols 0-7, kg=1: tile 2pp+1 cols 0-7, kg=2: tile 2pp cols 8-15, kg=3: tile 2pp+1
        // cols 8-15).  The gate arrives in that layout and is traded back the same way
        // (the swap is its own inverse), so loads and stores are 16-byte runs and a row's
        // 4 lanes cover 64 contiguous bytes.
        T* orow = out + (rowbase + p + iq) * ors + out_col + h * HD + gcol;
#pragma unroll
        for (int pp = 0; pp < NG; ++pp) {
          uint32_t gw[2][2] = {{0u, 0u}, {0u, 0u}};  // [tile of the pair][word]
          if constexpr (EPI) {
            const uint4 gr = graw[pp];
            const auto g0 = __builtin_amdgcn_permlane16_swap(gr.x, gr.z, false, false);
            const auto g1 = __builtin_amdgcn_permlane16_swap(gr.y, gr.w, false, false);
            gw[0][0] = g0[0], gw[0][1] = g1[0], gw[1][0] = g0[1], gw[1][1] = g1[1];
          }
          uint32_t ow[2][2];
#pragma unroll
          for (int hv = 0; hv < 2; ++hv) {
            const int vt = 2 * pp + hv;
            float o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const uint32_t gwr = gw[hv][r >> 1];
              o[r] = out_val(vt, r, __uint_as_float((r & 1) ? (gwr & 0xffff0000u) : (gwr << 16)));
            }
            ow[hv][0] = pack_bf16x2(o[0], o[1]);
            ow[hv][1] = pack_bf16x2(o[2], o[3]);
            if constexpr (EPI) {
              bf16_pair_sums(ow[hv][0], st_s, st_q);
              bf16_pair_sums(ow[hv][1], st_s, st_q);
            }
          }
          const auto s0 = __builtin_amdgcn_permlane16_swap(ow[0][0], ow[1][0], false, false);
          const auto s1 = __builtin_amdgcn_permlane16_swap(ow[0][1], ow[1][1], false, false);
          uint4 ov = make_uint4(s0[0], s1[0], s0[1], s1[1]);
          if constexpr (CHAIN) {  // 8 consecutive columns; z was loaded with them, a tile ahead
            {
              float zf[8], of[8];
              unpack16<T>(graw[pp], zf);
              unpack16<T>(ov, of);
#pragma unroll
              for (int e = 0; e < 8; ++e) of[e] *= zf[e] > 0.f ? 1.0f : fexp(zf[e]);
              ov = __builtin_bit_cast(uint4, pack_bf16x8(of));
            }
          }
          if (iq < tlen) *reinterpret_cast<uint4*>(orow + pp * 32) = ov;
        }
      } else if (iq < tlen) {
        T* orow = out + (rowbase + p + iq) * ors + out_col + h * HD + kg * 4;
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) {
          float gv[4] = {0.f, 0.f, 0.f, 0.f}, o[4];
          if constexpr (EPI) load4<T>(reinterpret_cast<const T*>(&graw[vt]), gv);
#pragma unroll
          for (int r = 0; r < 4; ++r) o[r] = out_val(vt, r, gv[r]);
          if constexpr (EPI) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float sv = rnd<T>(o[r]);
              st_s += sv;
              st_q = fmaf(sv, sv, st_q);
            }
          }
          if constexpr (CHAIN) {
            float z[4];
            load4<T>(reinterpret_cast<const T*>(&graw[vt]), z);
#pragma unroll
            for (int r = 0; r < 4; ++r) o[r] *= z[r] > 0.f ? 1.0f : fexp(z[r]);
          }
          store4<T>(orow + vt * 16, o);
        }
      }
      if constexpr (EPI) {
        if (row_stats != nullptr) {  // the row's 4 lanes l16 + 16 kg
          st_s = quad_group_sum(st_s);
          st_q = quad_group_sum(st_q);
          if (kg == 0 && iq < tlen)
            *reinterpret_cast<float2*>(row_stats + 2 * (h * stats_ps + rowbase + p + iq)) = make_float2(st_s, st_q);
        }
      }
      // next tile's gate (this tile's again after the last: a fixed load count)
      if constexpr (EPI || CHAIN) load_gate(p + tlen < p_end ? p + tlen : p);
    }

    // ---- state update: (W or A) <- gamma^tlen * (W or A) + K~^T V
    {
      const float gt = fexp2((float)tlen * lg2);
#pragma unroll
      for (int ov = 0; ov < OWN; ++ov) {
        const int vt = w + kWaves * ov;
        if (vt >= NVT) continue;
        Frag<T> bv[NJS];
#pragma unroll
        for (int ks = 0; ks < NJS; ++ks)
          frag_tok<T, HD, TC>(bv[ks], sm + LD::oV, vt * 16, 32 * ks, lane);
#pragma unroll
        for (int mt = 0; mt < NVT; ++mt) {
          f32x4_t acc;
          if constexpr (HAS_W) acc = stW[ov][mt] * gt;
          else acc = stA[ov][mt] * gt;
#pragma unroll
          for (int ks = 0; ks < NJS; ++ks) {
            Frag<T> a;
            frag_tok<T, HD, TC>(a, sm + LD::oKd, mt * 16, 32 * ks, lane);
            acc = mma(a, bv[ks], acc);
          }
          if constexpr (HAS_W) stW[ov][mt] = acc;
          else stA[ov][mt] = acc;
        }
      }
      if constexpr (HAS_W) {
        if (((p + tlen) % C) == 0) {
          const float gC = fexp2((float)C * lg2);
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

// Per (segment, head, batch): U_s = sum_{j in segment} gamma^(end-1-j) k~_j^T v_j, with k~
// from phi(k) (PHI) or k itself.  k starts at column k_col of each row, v v_off columns later.
template <typename T, int HD, int TC, bool PHI>
__global__ __launch_bounds__(kThreads, HD > 64 ? 2 : 4) void slot_state_kernel(const T* __restrict__ projs,
                                                              int64_t prs, int k_col, int v_off,
                                                              int L, const T* __restrict__ gamma,
                                                              int seg_rows, int nseg,
                                                              float* __restrict__ U) {
  using LD = Lds<T, HD, TC>;
  using TL = TileLoader<T, HD, TC, 1, 2>;
  __shared__ __attribute__((aligned(16))) T sm[LD::stTotal];
  constexpr int NVT = HD / 16;
  constexpr int NJS = TC / 32;
  constexpr int OWN = (NVT + kWaves - 1) / kWaves;

  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int l16 = lane & 15, kg = lane >> 4;
  const int h = blockIdx.x, seg = blockIdx.y, b = blockIdx.z, H = gridDim.x;
  const float lg2 = log2f(to_f<T>(gamma[h]));
  const int64_t rowbase = (int64_t)b * L;
  const int p_begin = seg * seg_rows;
  const int p_end = min(L, p_begin + seg_rows);
  const T* colbase = projs + k_col + h * HD;

  f32x4_t st[OWN][NVT];
#pragma unroll
  for (int ov = 0; ov < OWN; ++ov)
#pragma unroll
    for (int mt = 0; mt < NVT; ++mt) st[ov][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Two tiles in flight: the per-tile MFMA work is short, so one tile of prefetch would
  // leave each step waiting for a full memory round trip.  Prefetches past the segment
  // re-read the current tile, and the loop body always runs both steps (tlen = 0 makes a
  // step a no-op: zero tile, gamma^0 = 1), so every path issues the same loads in the same
  // order and the compiler's memory-counter waits stay exact.
  const TL loader(prs, {0, v_off}, tid);
  uint4 raw0[TL::NL], raw1[TL::NL];
  const T* tbase = colbase + rowbase * prs;
  // U_s is a decayed sum over the segment's rows, so the tiles need not follow chunks
  const int p1 = p_begin + TC < p_end ? p_begin + TC : p_begin;
  loader.load(raw0, tbase + (int64_t)p_begin * prs, min(TC, p_end - p_begin));
  loader.load(raw1, tbase + (int64_t)p1 * prs, min(TC, p_end - p1));

  auto step = [&](uint4 (&raw)[TL::NL], int p, int tlen) {
    __syncthreads();
    stage_tile<T, HD, TC, 1, 2, true, PHI>(raw, sm, tlen, lg2, tid);
    const int pn = p + 2 * TC < p_end ? p + 2 * TC : p;
    loader.load(raw, tbase + (int64_t)pn * prs, min(TC, p_end - pn));
    __syncthreads();
    const float gt = fexp2((float)tlen * lg2);
#pragma unroll
    for (int ov = 0; ov < OWN; ++ov) {
      const int vt = w + kWaves * ov;
      if (vt >= NVT) continue;
      Frag<T> bv[NJS];
#pragma unroll
      for (int ks = 0; ks < NJS; ++ks)
        frag_tok<T, HD, TC>(bv[ks], sm + LD::stV, vt * 16, 32 * ks, lane);
#pragma unroll
      for (int mt = 0; mt < NVT; ++mt) {
        f32x4_t acc = st[ov][mt] * gt;
#pragma unroll
        for (int ks = 0; ks < NJS; ++ks) {
          Frag<T> a;
          frag_tok<T, HD, TC>(a, sm + LD::stKd, mt * 16, 32 * ks, lane);
          acc = mma(a, bv[ks], acc);
        }
        st[ov][mt] = acc;
      }
    }
  };
  for (int p = p_begin; p < p_end; p += 2 * TC) {
    step(raw0, p, min(TC, p_end - p));
    const bool second = p + TC < p_end;
    step(raw1, second ? p + TC : p, second ? min(TC, p_end - p - TC) : 0);
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
  const int64_t bh = (int64_t)b * H + h;
  const T graw = gamma[h];
  const float* u = U + bh * nseg * HD2 + e;
  float* o = Ain + bh * nseg * HD2 + e;
  // Segments in batches of kU whose loads are all in flight before the recurrence uses them.
  // The first batch is straight-line code issued before S0 is loaded and gamma used, so no
  // wait precedes its loads; U[s] is needed only for s + 1 < nseg.
  constexpr int kU = 32;
  float uu[kU];
#pragma unroll
  for (int k = 0; k < kU; ++k) uu[k] = (k + 1 < nseg) ? u[(int64_t)k * HD2] : 0.f;
  float a = S0 ? S0[bh * HD2 + e] : 0.f;
  const float gs = fexp2((float)seg_len * log2f(to_f<T>(graw)));
#pragma unroll
  for (int k = 0; k < kU; ++k) {
    if (k < nseg) {
      o[(int64_t)k * HD2] = a;
      a = a * gs + uu[k];
    }
  }
  for (int s = kU; s < nseg; s += kU) {
#pragma unroll
    for (int k = 0; k < kU; ++k) uu[k] = (s + k + 1 < nseg) ? u[(int64_t)(s + k) * HD2] : 0.f;
#pragma unroll
    for (int k = 0; k < kU; ++k) {
      if (s + k < nseg) {
        o[(int64_t)(s + k) * HD2] = a;
        a = a * gs + uu[k];
      }
    }
  }
}

}  // namespace

namespace hdcm_slot {
// Launch plan shared by the translation units of the slot kernels.
struct SlotPlan {
  int HD, TC, seg_rows, nseg, cshift;
  bool has_w;
  bool conf;  // chunk-confined tiles: C neither divides TC nor is a multiple of it
};
}  // namespace hdcm_slot

namespace {
using hdcm_slot::SlotPlan;

// Supported head dims: multiples of 16 up to 128.
inline bool slot_head_dim_ok(int64_t hd) { return hd >= 16 && hd <= 128 && hd % 16 == 0; }

int slot_plan(int64_t B, int64_t L, int64_t dm, int64_t H, int64_t C, int dtype, SlotPlan* pl) {
  if (dtype != HDCM_F32 && dtype != HDCM_BF16) return HDCM_EUNSUPPORTED;
  if (B < 0 || L < 0 || dm <= 0 || H <= 0 || C <= 0 || dm % H) return HDCM_EINVAL;
  const int64_t HD = dm / H;
  if (!slot_head_dim_ok(HD)) return HDCM_EUNSUPPORTED;
  const int TC = dtype == HDCM_BF16 ? 64 : 32;
  if (L % C) return HDCM_EINVAL;
  if (C > ((int64_t)1 << 30)) return HDCM_EUNSUPPORTED;
  // C dividing TC (a power of two below it): tiles of TC rows hold whole chunks; any other C:
  // chunk-confined tiles (cshift = 31), ceil(C/TC) per chunk
  int cshift = 31;
  if (C < TC && TC % C == 0) {
    cshift = 0;
    while ((1 << cshift) < C) ++cshift;
  }
  if (B > 65535 || H > 65535) return HDCM_EUNSUPPORTED;
  const int64_t tiles = (L + TC - 1) / TC;
  int64_t st = hdcm_option_value(HDCM_OPT_SLOT_SEG_TILES);  // 0: automatic
  if (st == 0) {
    const int64_t bh = B * H > 0 ? B * H : 1;
    const int64_t want = (kTargetWorkgroups + bh - 1) / bh;
    st = (tiles + want - 1) / want;
    if (st < kMinSegTiles) st = kMinSegTiles;
  }
  if (st < 1) st = 1;
  // segments start on chunk boundaries: whole TC-row tiles (C dividing TC), else whole chunks
  int64_t seg_rows;
  if (cshift < 31) {
    seg_rows = st * TC;
  } else {
    const int64_t tpc = (C + TC - 1) / TC;  // tiles per chunk
    seg_rows = (st + tpc - 1) / tpc * C;
  }
  if (L > 0 && seg_rows > L) seg_rows = cshift < 31 ? tiles * TC : L;
  if (seg_rows < 1) seg_rows = 1;
  pl->HD = (int)HD;
  pl->TC = TC;
  pl->seg_rows = (int)(seg_rows > ((int64_t)1 << 30) ? ((int64_t)1 << 30) : seg_rows);
  pl->nseg = (int)((L + seg_rows - 1) / seg_rows);
  if (pl->nseg < 1) pl->nseg = 1;
  pl->cshift = cshift;
  pl->has_w = C > TC;
  pl->conf = cshift >= 31 && C % TC != 0;
  if (pl->nseg > 65535 || L > ((int64_t)1 << 30)) return HDCM_EUNSUPPORTED;
  return HDCM_OK;
}

size_t slot_ws_bytes(int64_t B, int64_t H, const SlotPlan& pl) {
  return (size_t)2 * B * H * pl.nseg * pl.HD * pl.HD * sizeof(float);
}

// k at column k_col of each row, v v_off columns after k; PHI as in the kernels.
template <typename T, int HD, bool PHI>
int launch_state(const void* base, int64_t prs, int64_t k_col, int64_t v_off, const void* gamma,
                 const float* S0, void* ws, int64_t B, int64_t L, int64_t H, const SlotPlan& pl,
                 hipStream_t s) {
  constexpr int TC = TileOf<T>::value;
  float* U = (float*)ws;
  float* Ain = U + (size_t)B * H * pl.nseg * HD * HD;
  if (pl.nseg > 1) {
    HDCM_LAUNCH((slot_state_kernel<T, HD, TC, PHI>), dim3((unsigned)H, pl.nseg - 1, (unsigned)B),
                       dim3(kThreads), 0, s, (const T*)base, prs, (int)k_col, (int)v_off, (int)L,
                       (const T*)gamma, pl.seg_rows, pl.nseg, U);
    const int st = hdcm_launch_status();
    if (st) return st;
  }
  HDCM_LAUNCH((slot_scan_kernel<T>), dim3((HD * HD + kThreads - 1) / kThreads, (unsigned)H, (unsigned)B),
                     dim3(kThreads), 0, s, U, S0, Ain, (const T*)gamma, HD * HD, pl.nseg,
                     pl.seg_rows);
  return hdcm_launch_status();
}

// q at column q_col of each row; k, v and the gate k_off, v_off, g_off columns after q.
template <typename T, int HD, bool PHI, bool EPI, bool CHAIN = false>
int launch_gate(const void* base, int64_t prs, int64_t q_col, int64_t k_off, int64_t v_off, int64_t g_off,
                const void* gamma, const void* gn_w, const void* gn_b, float gn_eps, const void* ws, void* out,
                int64_t ors, int64_t out_col, float* S_final, float* row_stats, int64_t stats_ps, int64_t B,
                int64_t L, int64_t H, int64_t C, const SlotPlan& pl, hipStream_t s, const void* zb = nullptr,
                int64_t zrs = 0) {
  constexpr int TC = TileOf<T>::value;
  const float* Ain = (const float*)ws + (size_t)B * H * pl.nseg * HD * HD;
  // heads vary fastest so the workgroups that run together read the same rows of projs
  dim3 grid((unsigned)H, pl.nseg, (unsigned)B);
  // 16-byte output runs need 16-byte aligned rows and columns (bf16 only; fp32 always has them)
  // (with CHAIN the z rows must allow the same 16-byte runs)
  const bool pairs = sizeof(T) == 2 && ((uintptr_t)out % 16) == 0 && out_col % 8 == 0 && ors % 8 == 0 &&
                     (!CHAIN || (((uintptr_t)zb % 16) == 0 && zrs % 8 == 0));
#define HDCM_GATE_LAUNCH(W, P, CF)                                                                          \
  HDCM_LAUNCH((slot_gate_kernel<T, HD, TC, W, P, PHI, EPI, CHAIN, CF>), grid, dim3(kThreads), 0, s,    \
                     (const T*)base, prs, (int)q_col, (int)k_off, (int)v_off, (int)g_off, (int)L, (int)C,  \
                     pl.cshift, (const T*)gamma, (const T*)gn_w, (const T*)gn_b, gn_eps, Ain, pl.seg_rows,   \
                     pl.nseg, (T*)out, ors, (int)out_col, S_final, row_stats, stats_ps, (const T*)zb, zrs)
  // chunk-confined tiles (rare chunk sizes) run with the 8-byte output runs only
  if (pl.conf) {
    if (pl.has_w) HDCM_GATE_LAUNCH(true, false, true);
    else HDCM_GATE_LAUNCH(false, false, true);
  } else if (pl.has_w) {
    if (pairs) HDCM_GATE_LAUNCH(true, true, false);
    else HDCM_GATE_LAUNCH(true, false, false);
  } else {
    if (pairs) HDCM_GATE_LAUNCH(false, true, false);
    else HDCM_GATE_LAUNCH(false, false, false);
  }
#undef HDCM_GATE_LAUNCH
  return hdcm_launch_status();
}

int check_projs(const void* projs, int64_t prs, int64_t q_col, int64_t dm, int dtype, bool empty) {
  const int E = 16 / hdcm_elt_size(dtype);
  if (!projs && !empty) return HDCM_EINVAL;  // empty inputs (B or L zero) may have no storage
  if (q_col < 0 || prs < q_col + 4 * dm) return HDCM_EINVAL;
  if (!hdcm_aligned16(projs) || prs % E || q_col % E || dm % E) return HDCM_EALIGN;
  return HDCM_OK;
}

}  // namespace

// The plain attention pass (hdcm_slot_attend_fwd) for one dtype, after argument checks; its
// instantiations live in their own translation units (slot_attend.hip: bf16,
// slot_attend_f32.hip: fp32) so the slot kernels compile in parallel.
namespace hdcm_slot {
int attend_launch_bf16(const void* base, int64_t row_stride, int64_t q_col, int64_t k_col, int64_t v_col,
                       const void* gamma, int phi, void* ws, void* out, int64_t out_row_stride, int64_t out_col,
                       const void* chain, int64_t chain_row_stride, int64_t B, int64_t L, int64_t H, int64_t C,
                       const SlotPlan& pl, hipStream_t s);
int attend_launch_f32(const void* base, int64_t row_stride, int64_t q_col, int64_t k_col, int64_t v_col,
                      const void* gamma, int phi, void* ws, void* out, int64_t out_row_stride, int64_t out_col,
                      const void* chain, int64_t chain_row_stride, int64_t B, int64_t L, int64_t H, int64_t C,
                      const SlotPlan& pl, hipStream_t s);
}  // namespace hdcm_slot

