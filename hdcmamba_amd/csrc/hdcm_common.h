// Shared device helpers for the HdcMamba gfx950 kernels.
//
// Element types: activations are either fp32 (`float`) or bf16 stored as raw
// `uint16_t` bits.  All arithmetic is fp32; bf16 values are produced with
// round-to-nearest-even, the rounding torch and the MFMA operand path use.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hdcm.h"

// ------------------------------------------------------------ launch timing hook
// hdcm_time_launches(starts, stops, n) (api.hip) arms the calling thread: the k-th kernel it
// launches through HDCM_LAUNCH (k < n) records starts[k] when it begins and stops[k] when it
// ends, from the dispatch's own timestamps (hipExtLaunchKernel).  Launches past n, and all
// launches of an unarmed thread, are plain hipLaunchKernelGGL.
struct HdcmTiming {
  void* const* start;
  void* const* stop;
  int n, used;
};
extern thread_local HdcmTiming hdcm_timing_slot;

// Launch options (hdcm_set_option, api.hip): their values when the library loaded come from
// the environment, read once; a launch reads the value current when it is issued.
int hdcm_option_value(int option);

#define HDCM_LAUNCH(kernel, grid, block, shmem, stream, ...)                                      \
  do {                                                                                            \
    if (hdcm_timing_slot.used < hdcm_timing_slot.n) {                                             \
      const int k_ = hdcm_timing_slot.used++;                                                     \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream,                                   \
                            (hipEvent_t)hdcm_timing_slot.start[k_],                               \
                            (hipEvent_t)hdcm_timing_slot.stop[k_], 0u, __VA_ARGS__);              \
    } else {                                                                                      \
      hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                        \
    }                                                                                             \
  } while (0)

namespace hdcm {

typedef uint16_t bf16_t;
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float bf2f(bf16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// Round-to-nearest-even through the gfx950 hardware conversion (v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// Fast transcendentals: single v_exp_f32 / v_log_f32 / v_rcp_f32 instructions (about
// 1 ulp on the instruction's own argument).
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fexp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
__device__ __forceinline__ float flog(float x) { return __builtin_amdgcn_logf(x) * kLn2; }
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }

template <typename T> __device__ __forceinline__ float to_f(T v);
template <> __device__ __forceinline__ float to_f<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f<bf16_t>(bf16_t v) { return bf2f(v); }

template <typename T> __device__ __forceinline__ T from_f(float v);
template <> __device__ __forceinline__ float from_f<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16_t from_f<bf16_t>(float v) { return f2bf(v); }

// Round to the storage type and back (identity for fp32).
template <typename T> __device__ __forceinline__ float rnd(float v) { return to_f<T>(from_f<T>(v)); }

// Elements per 16-byte vector.
template <typename T> struct Vec { static constexpr int N = 16 / sizeof(T); };

// ------------------------------------------------------- 16-byte vector I/O
template <typename T> __device__ __forceinline__ void load16(const T* p, float* out);
template <> __device__ __forceinline__ void load16<float>(const float* p, float* out) {
  float4 v = *reinterpret_cast<const float4*>(p);
  out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
}
template <> __device__ __forceinline__ void load16<bf16_t>(const bf16_t* p, float* out) {
  uint4 v = *reinterpret_cast<const uint4*>(p);
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

template <typename T> __device__ __forceinline__ void store16(T* p, const float* in);
template <> __device__ __forceinline__ void store16<float>(float* p, const float* in) {
  *reinterpret_cast<float4*>(p) = make_float4(in[0], in[1], in[2], in[3]);
}
// Two fp32 values rounded (nearest even) into one packed bf16 pair: a single
// v_cvt_pk_bf16_f32 with both sources.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b16x2 __attribute__((ext_vector_type(2)));
  const f32x2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, b16x2));
}

// The 16-byte word store16 writes for these values (they, rounded to T as stored).
template <typename T> __device__ __forceinline__ uint4 pack16(const float* in);
template <> __device__ __forceinline__ uint4 pack16<float>(const float* in) {
  return make_uint4(__float_as_uint(in[0]), __float_as_uint(in[1]), __float_as_uint(in[2]), __float_as_uint(in[3]));
}
template <> __device__ __forceinline__ uint4 pack16<bf16_t>(const float* in) {
  return make_uint4(pack_bf16x2(in[0], in[1]), pack_bf16x2(in[2], in[3]), pack_bf16x2(in[4], in[5]),
                    pack_bf16x2(in[6], in[7]));
}

template <> __device__ __forceinline__ void store16<bf16_t>(bf16_t* p, const float* in) {
  *reinterpret_cast<uint4*>(p) = pack16<bf16_t>(in);
}

// Adds a packed bf16 pair and its squares to s and q (fp32 accumulation of the exact
// products, v_dot2_f32_bf16).
__device__ __forceinline__ void bf16_pair_sums(uint32_t w, float& s, float& q) {
  typedef __bf16 b16x2 __attribute__((ext_vector_type(2)));
  const b16x2 p = __builtin_bit_cast(b16x2, w), one = __builtin_bit_cast(b16x2, 0x3f803f80u);
  s = __builtin_amdgcn_fdot2_f32_bf16(p, one, s, false);
  q = __builtin_amdgcn_fdot2_f32_bf16(p, p, q, false);
}

// store16 that also adds the stored values (as rounded to T) and their squares to s and q:
// the row statistics a later row LayerNorm needs, taken where the values are produced.
template <typename T> __device__ __forceinline__ void store16_sums(T* p, const float* in, float& s, float& q);
template <> __device__ __forceinline__ void store16_sums<float>(float* p, const float* in, float& s, float& q) {
  store16<float>(p, in);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    s += in[e];
    q = fmaf(in[e], in[e], q);
  }
}
template <> __device__ __forceinline__ void store16_sums<bf16_t>(bf16_t* p, const float* in, float& s, float& q) {
  uint4 v;
  v.x = pack_bf16x2(in[0], in[1]);
  v.y = pack_bf16x2(in[2], in[3]);
  v.z = pack_bf16x2(in[4], in[5]);
  v.w = pack_bf16x2(in[6], in[7]);
  *reinterpret_cast<uint4*>(p) = v;
  bf16_pair_sums(v.x, s, q);
  bf16_pair_sums(v.y, s, q);
  bf16_pair_sums(v.z, s, q);
  bf16_pair_sums(v.w, s, q);
}

// Raw (unconverted) 16-byte loads, for staging data whose conversion happens later.
__device__ __forceinline__ uint4 ldg16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

template <typename T> __device__ __forceinline__ void unpack16(uint4 v, float* out);
template <> __device__ __forceinline__ void unpack16<float>(uint4 v, float* out) {
  out[0] = __uint_as_float(v.x); out[1] = __uint_as_float(v.y);
  out[2] = __uint_as_float(v.z); out[3] = __uint_as_float(v.w);
}
template <> __device__ __forceinline__ void unpack16<bf16_t>(uint4 v, float* out) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

// ------------------------------------------------------------ wave reductions
// Butterfly over all 64 lanes; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Sum over all 64 lanes on DPP lane moves (quad swaps, half-row and row mirrors, then
// row_bcast 15/31 fold the rows into lane 63), read into a wave-uniform scalar.
__device__ __forceinline__ float wave_total(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));   // quad [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));   // quad [2,3,0,1]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));  // row_half_mirror
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false));  // row_mirror
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, false));  // row_bcast:15
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xc, 0xf, false));  // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum over aligned groups of GL lanes (GL a power of two up to 64); every lane of a group
// receives the group's total.  Quad swaps, then the half-row and row mirrors (once the
// smaller groups hold equal values a mirror pairs each lane with the other half), then
// cross-row shuffles.
template <int GL>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(GL >= 1 && GL <= 64 && (GL & (GL - 1)) == 0, "group of 2^k lanes");
  if (GL >= 2) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));
  if (GL >= 4) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));
  if (GL >= 8) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));
  if (GL >= 16) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false));
  if (GL >= 32) v += __shfl_xor(v, 16, kWave);
  if (GL >= 64) v += __shfl_xor(v, 32, kWave);
  return v;
}

// Sum over the four lanes l, l^16, l^32, l^48 (the row groups of an MFMA C/D tile), on the
// gfx950 lane-row swaps (VALU, no LDS traffic).  v_permlane16_swap(a, b) returns
// (a.r0, b.r0, a.r2, b.r2) and (a.r1, b.r1, a.r3, b.r3) for 16-lane rows r0..r3, so with
// a = b = v their sum is r0+r1 in rows 0-1 and r2+r3 in rows 2-3; v_permlane32_swap returns
// (a.r0, a.r1, b.r0, b.r1) and (a.r2, a.r3, b.r2, b.r3), whose sum adds the two halves.
// Every lane gets (x0 + x1) + (x2 + x3), bit for bit.
__device__ __forceinline__ float quad_group_sum(float v) {
  const unsigned u = __float_as_uint(v);
  const auto h = __builtin_amdgcn_permlane16_swap(u, u, true, false);  // fetch inactive lanes too
  const float s = __uint_as_float(h[0]) + __uint_as_float(h[1]);
  const unsigned us = __float_as_uint(s);
  const auto q = __builtin_amdgcn_permlane32_swap(us, us, true, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// softplus with the threshold 20 of F.softplus: x above it, log(1 + exp(x)) below.
// Feature map elu(z)+1 of the slot memory: exp(min(z,0)) + max(z,0), which is z+1 for z>0
// and exp(z) otherwise.  min and max against +0 are taken on the bit patterns as signed
// integers (IEEE floats of either sign order like their patterns), so no canonicalising
// v_max is needed on inputs that were bit-cast from bf16 storage.
__device__ __forceinline__ float phi_f(float z) {
  const int b = __float_as_int(z);
  return fexp(__int_as_float(min(b, 0))) + __int_as_float(max(b, 0));
}
__device__ __forceinline__ float softplus20(float v) { return v > 20.0f ? v : flog(1.0f + fexp(v)); }

// One Hillis-Steele step of the (a, u) scan: combine with the pair fetched by the DPP
// control CTRL; lanes whose source is out of range or masked off fetch the identity (1, 0).
template <int CTRL, int ROW_MASK, int NC>
__device__ __forceinline__ void scan_step_dpp(float (&a)[NC], float (&u)[NC]) {
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const float ap = __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(1.0f), __float_as_int(a[c]), CTRL, ROW_MASK, 0xf, false));
    const float up = __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(0.0f), __float_as_int(u[c]), CTRL, ROW_MASK, 0xf, false));
    u[c] = a[c] * up + u[c];
    a[c] = a[c] * ap;
  }
}

// Inclusive scans over the wave's 64 lanes (lane order) of NC independent (a, u) pair
// streams under (a1, u1) then (a2, u2) = (a1*a2, a2*u1 + u2), on DPP lane moves:
// row_shr 1, 2, 4, 8 scan each 16-lane row; row_bcast 15 then folds row 0 into row 1 and
// row 2 into row 3, and row_bcast 31 folds rows 0-1 into rows 2-3.
template <int NC>
__device__ __forceinline__ void scan_pairs(float (&a)[NC], float (&u)[NC]) {
  scan_step_dpp<0x111, 0xf>(a, u);  // row_shr:1
  scan_step_dpp<0x112, 0xf>(a, u);  // row_shr:2
  scan_step_dpp<0x114, 0xf>(a, u);  // row_shr:4
  scan_step_dpp<0x118, 0xf>(a, u);  // row_shr:8
  scan_step_dpp<0x142, 0xa>(a, u);  // row_bcast:15 into rows 1 and 3
  scan_step_dpp<0x143, 0xc>(a, u);  // row_bcast:31 into rows 2 and 3
}

// ------------------------------------------------------------- MFMA fragments
// A 16x16 MFMA tile step contracts K=32.  A lane owns 8 contraction slots s=0..7 of
// one row (A operand) or column (B operand).  For bf16 the 8 slots feed one
// v_mfma_f32_16x16x32_bf16; for fp32 they feed eight v_mfma_f32_16x16x4_f32, slot s
// going to the s-th instruction.  Either way lane group g=lane/16 and slot s name
// the same contraction index in the A and the B fragment, so any bijection
// (g,s) -> k used consistently for both operands yields the full K=32 sum.
//
// Output layout (both instruction families): lane l holds D[4*(l/16)+r][l%16], r=0..3.
template <typename T> struct Frag;
template <> struct Frag<bf16_t> { bf16x8_t v; };
template <> struct Frag<float> { float v[8]; };

__device__ __forceinline__ f32x4_t mma(const Frag<bf16_t>& a, const Frag<bf16_t>& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mma(const Frag<float>& a, const Frag<float>& b, f32x4_t c) {
#pragma unroll
  for (int s = 0; s < 8; ++s) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[s], b.v[s], c, 0, 0, 0);
  return c;
}

// 8 consecutive elements (slots 0..7) from LDS.
__device__ __forceinline__ void frag_load8(Frag<bf16_t>& f, const bf16_t* p) {
  f.v = *reinterpret_cast<const bf16x8_t*>(p);
}
__device__ __forceinline__ void frag_load8(Frag<float>& f, const float* p) {
  float4 a = *reinterpret_cast<const float4*>(p);
  float4 b = *reinterpret_cast<const float4*>(p + 4);
  f.v[0] = a.x; f.v[1] = a.y; f.v[2] = a.z; f.v[3] = a.w;
  f.v[4] = b.x; f.v[5] = b.y; f.v[6] = b.z; f.v[7] = b.w;
}
// Slots 0..3 from p0 and slots 4..7 from p1 (4 consecutive elements each).
__device__ __forceinline__ void frag_load4x2(Frag<bf16_t>& f, const bf16_t* p0, const bf16_t* p1) {
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  bf16x4_t a = *reinterpret_cast<const bf16x4_t*>(p0);
  bf16x4_t b = *reinterpret_cast<const bf16x4_t*>(p1);
  f.v = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ void frag_load4x2(Frag<float>& f, const float* p0, const float* p1) {
  float4 a = *reinterpret_cast<const float4*>(p0);
  float4 b = *reinterpret_cast<const float4*>(p1);
  f.v[0] = a.x; f.v[1] = a.y; f.v[2] = a.z; f.v[3] = a.w;
  f.v[4] = b.x; f.v[5] = b.y; f.v[6] = b.z; f.v[7] = b.w;
}
// 8 fp32 values rounded (nearest even) into 8 bf16: four paired v_cvt_pk_bf16_f32.
__device__ __forceinline__ bf16x8_t pack_bf16x8(const float* x) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 u = {pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]), pack_bf16x2(x[4], x[5]),
                   pack_bf16x2(x[6], x[7])};
  return __builtin_bit_cast(bf16x8_t, u);
}
// The 8 values of a bf16 vector as fp32 (exact).
__device__ __forceinline__ void unpack_bf16x8(bf16x8_t v, float* x) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 u = __builtin_bit_cast(u32x4, v);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(u[i] << 16);
    x[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
}
// Build a fragment from 8 fp32 values, rounding to the operand type.
__device__ __forceinline__ void frag_from_f32(Frag<bf16_t>& f, const float* x) { f.v = pack_bf16x8(x); }
__device__ __forceinline__ void frag_from_f32(Frag<float>& f, const float* x) {
#pragma unroll
  for (int s = 0; s < 8; ++s) f.v[s] = x[s];
}

// ------------------------------------------------------ fixed-order column sums
// Parameter gradients are summed over rows in two steps: each workgroup of a row pass leaves
// one row of partial sums, then colsum_kernel adds the partial rows.  Column c of out (c <
// ncols) is the sum over k < nk of part[base(c) + k * kstride], base(c) = (c / cgroup) *
// gstride + c % cgroup; thread (x, j) of a 64-column x 16-row workgroup adds rows k = j,
// j + 16, ... and the 16 sums are then added in order of j, so the result does not depend on
// scheduling.  Columns c < nsplit go to out0[c], the others to out1[c - nsplit].
constexpr int kSumCols = 64, kSumRows = 16;
__global__ __launch_bounds__(kSumCols* kSumRows) static void colsum_kernel(
    const float* __restrict__ part, int64_t kstride, int nk, int ncols, int cgroup, int64_t gstride,
    float* __restrict__ out0, int nsplit, float* __restrict__ out1) {
  __shared__ float acc[kSumRows][kSumCols + 1];
  const int x = threadIdx.x % kSumCols, j = threadIdx.x / kSumCols;
  const int c = blockIdx.x * kSumCols + x;
  float s = 0.f;
  if (c < ncols) {
    const int64_t base = (int64_t)(c / cgroup) * gstride + c % cgroup;
    for (int k = j; k < nk; k += kSumRows) s += part[base + (int64_t)k * kstride];
  }
  acc[j][x] = s;
  __syncthreads();
  if (j == 0 && c < ncols) {
    float t = 0.f;
#pragma unroll
    for (int r = 0; r < kSumRows; ++r) t += acc[r][x];
    if (c < nsplit) out0[c] = t;
    else out1[c - nsplit] = t;
  }
}

// Host-side dtype mapping.
template <typename T> struct DtypeOf;
template <> struct DtypeOf<float> { static constexpr int value = HDCM_F32; };
template <> struct DtypeOf<bf16_t> { static constexpr int value = HDCM_BF16; };

}  // namespace hdcm

// ------------------------------------------------------------ host-side checks
#define HDCM_CHECK_ARG(cond, code) \
  do {                             \
    if (!(cond)) return (code);    \
  } while (0)

static inline bool hdcm_aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
static inline int hdcm_elt_size(int dtype) { return dtype == HDCM_F32 ? 4 : 2; }

static inline int hdcm_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? HDCM_OK : HDCM_ELAUNCH;
}

// Launch colsum_kernel (see there) on `s`; nk == 0 writes zeros.
static inline int hdcm_colsum(const float* part, int64_t kstride, int nk, int ncols, int cgroup, int64_t gstride,
                              float* out0, int nsplit, float* out1, hipStream_t s) {
  HDCM_LAUNCH(hdcm::colsum_kernel,dim3((unsigned)((ncols + hdcm::kSumCols - 1) / hdcm::kSumCols)),
                     dim3(hdcm::kSumCols * hdcm::kSumRows), 0, s, part, kstride, nk, ncols, cgroup, gstride, out0,
                     nsplit, out1);
  return hdcm_launch_status();
}
