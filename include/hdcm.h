/*
 * hdcm.h -- C ABI of libhdcmamba_hip.so, the gfx950 (MI355X) kernels of the
 * HdcMamba block forward.
 *
 * Conventions
 *  - Every pointer is device memory owned by the caller.  The library never
 *    allocates, frees or synchronises; scratch space comes in through `ws`.
 *  - Activation tensors are row-major with unit element stride inside a row.
 *    Row strides are given in elements.  Rows of a [B,L,*] tensor are indexed
 *    b*L + t unless a separate batch stride is taken.  Every pointer and every
 *    row stride must keep rows 16-byte aligned (128-bit loads and stores).
 *  - `dtype` (hdcm_dtype) applies to every activation and parameter pointer of
 *    a call; recurrent states (`h0`, `h_final`, `S0`, `S_final`) are fp32.
 *  - `stream` is a hipStream_t; all work is ordered on it.  Calls on distinct
 *    streams with distinct buffers may run concurrently.
 *  - Functions return an hdcm_status.  Arguments are validated before any
 *    HIP call, so a failed validation has no side effect.
 *  - Empty inputs (a zero batch, sequence or row count) are valid: their data
 *    pointers may be NULL and their strides are not checked.  Nothing is read or
 *    written, except that gradients of parameters are set to zero.
 *
 * Reference: N01N9/hdcmamba launches Triton kernels from Python
 * (hdcmamba/model.py); each entry point below names the launch it replaces.
 */
#ifndef HDCM_H_
#define HDCM_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum { HDCM_F32 = 0, HDCM_BF16 = 1 } hdcm_dtype;

typedef enum {
  HDCM_OK = 0,
  HDCM_EINVAL = -1,       /* null pointer, bad shape or stride */
  HDCM_EALIGN = -2,       /* pointer or row stride not 16-byte aligned */
  HDCM_EUNSUPPORTED = -3, /* valid but not built: dtype/head_dim/chunk combination */
  HDCM_ELAUNCH = -4,      /* a HIP launch reported an error */
  HDCM_EWORKSPACE = -5,   /* workspace missing or smaller than required */
  HDCM_ETOOBIG = -6       /* input larger than a no-allocation entry point's fixed scratch */
} hdcm_status;

/* 2: hdcm_ssm_fwd and hdcm_slot_gate_fwd take row_stats and its part stride; the scan's
 *    workspace contract (zero before its first use, then kept between calls); launch options. */
#define HDCM_ABI_VERSION 2

int hdcm_abi_version(void);
const char* hdcm_strerror(int status);

/*
 * Kernel timing for measurement harnesses.  Arms the calling thread: the k-th kernel
 * (k < n) that the following hdcm_* calls of this thread launch records start_events[k] when
 * it begins and stop_events[k] when it ends (hipEvent_t handles, created by the caller),
 * from the dispatch's own begin/end timestamps (hipExtLaunchKernel), so no event packets
 * enter the stream.  The arrays must stay valid while armed; n = 0 disarms.
 * hdcm_timed_launch_count returns how many launches have recorded events since arming.
 * Not for calls made under stream capture.
 * No counterpart in the reference (benchmark.py:165-192 times whole forwards with
 * torch.cuda.synchronize around them).
 */
int hdcm_time_launches(void* const* start_events, void* const* stop_events, int n);
int hdcm_timed_launch_count(void);

/*
 * Launch options, for tests and tuning.  Their values when the library loads come from the
 * environment variables named below, read once; hdcm_set_option changes one for every later
 * launch of the process (a recorded graph keeps the values current at its capture).
 *  HDCM_OPT_SSM_SPIN_ROUNDS (env HDCM_SSM_SPIN_ROUNDS, default 256): polling rounds of the
 *    scan's look-back before a workgroup computes a missing earlier tile total itself
 *    (0 forces that path).  Results do not depend on it.
 *  HDCM_OPT_SLOT_SEG_TILES (env HDCM_SLOT_SEG_TILES, default 0 = automatic): row tiles per
 *    segment of the slot kernels.  Results do not depend on it beyond fp32 rounding.
 *  HDCM_OPT_SKINNY_COLS8_MAX_N (env HDCM_SKINNY_COLS8_MAX_N, default 4096): skinny GEMM
 *    outputs (hdcm_skinny_gemm_fwd, hdcm_rowln_gemm_fwd at <= 16 rows) of 2048 up to this
 *    many columns run 8 output columns per workgroup instead of 16 (0 switches it off).
 *    Results do not depend on it.
 *  HDCM_OPT_SKINNY_FOLD_TAIL (env HDCM_SKINNY_FOLD_TAIL, default 1): skinny GEMM outputs
 *    (N >= 2048, no folded LayerNorm) with more 16- or 8-column tiles than workgroups fit on
 *    the GPU at once, but at most twice as many, run one round of workgroups, the first ones
 *    taking a second tile, instead of a second round (0 switches it off).  Results do not
 *    depend on it.
 *  HDCM_OPT_STEP_SPIN_ROUNDS (env HDCM_STEP_SPIN_ROUNDS, default 65536): polling rounds of
 *    hdcm_norm_conv_in_proj_step_fwd's GEMM workgroups for the conv rows before they count a
 *    timeout in the workspace header and go on (their outputs are then not valid).
 * hdcm_set_option returns HDCM_EINVAL for an unknown option or a value out of range
 * (0 .. 2^20; SKINNY_COLS8_MAX_N 0 .. 2^30; SKINNY_FOLD_TAIL 0 .. 1; STEP_SPIN_ROUNDS 0 .. 2^24);
 * hdcm_get_option returns the current value (0 for an unknown one).
 * No counterpart in the reference (its launch table, model.py:12-19, is fixed).
 */
typedef enum {
  HDCM_OPT_SSM_SPIN_ROUNDS = 1,
  HDCM_OPT_SLOT_SEG_TILES = 2,
  HDCM_OPT_SKINNY_COLS8_MAX_N = 3,
  HDCM_OPT_SKINNY_FOLD_TAIL = 4,
  HDCM_OPT_STEP_SPIN_ROUNDS = 5
} hdcm_option;
int hdcm_set_option(int option, int value);
int hdcm_get_option(int option);

/*
 * LayerNorm over D (biased variance, eps) followed by the causal depthwise
 * conv of width 4: out[t] = sum_k LN(x)[t-3+k] * conv_w[:,k] + conv_b, with
 * LN rows t<0 equal to ln_b (LayerNorm of a zero row).
 * x, out: [B,L,D]; ln_w, ln_b, conv_b: [D]; conv_w: [D,4] contiguous.
 * Needs D % (16/elt_size) == 0 and D/(16/elt_size) <= 768 (bf16 D <= 6144,
 * fp32 D <= 3072).
 * Replaces: FusedNormConv1dFunction.forward -> _fused_norm_conv_fwd_kernel
 *           (hdcmamba/model.py:128-146, kernel model.py:22-72).
 */
int hdcm_norm_conv_fwd(const void* x, int64_t x_batch_stride, int64_t x_row_stride,
                       const void* ln_w, const void* ln_b, const void* conv_w, const void* conv_b,
                       void* out, int64_t out_batch_stride, int64_t out_row_stride,
                       int64_t B, int64_t L, int64_t D, float eps, int dtype, void* stream);

/*
 * Gradients of hdcm_norm_conv_fwd for grad_out = dL/dout [B,L,D] (strides as x): dx
 * [B,L,D] in the activation dtype, and fp32 d_ln_w [D], d_ln_b [D], d_conv_w [D,4],
 * d_conv_b [D].  Exact gradients of the forward, including the ln_b terms through the
 * LayerNorm of the zero rows before the sequence start; parameter gradients are summed in
 * a fixed order (deterministic).  ws: hdcm_norm_conv_bwd_workspace_bytes(B, L, D) bytes,
 * 256-byte aligned.  Needs D % (16/elt_size) == 0 and D/(16/elt_size) <= 768 (bf16
 * D <= 6144, fp32 D <= 3072: the forward's limits).
 * Replaces: FusedNormConv1dFunction.backward -> _fused_norm_conv_bwd_kernel
 *           (hdcmamba/model.py:149-166, kernel model.py:74-124), which omits the ln_b
 *           terms of d_conv_w and d_ln_b and uses bf16-rounded row statistics.
 */
size_t hdcm_norm_conv_bwd_workspace_bytes(int64_t B, int64_t L, int64_t D);
int hdcm_norm_conv_bwd(const void* grad_out, int64_t g_batch_stride, int64_t g_row_stride,
                       const void* x, int64_t x_batch_stride, int64_t x_row_stride, const void* ln_w,
                       const void* ln_b, const void* conv_w, void* dx, int64_t dx_batch_stride,
                       int64_t dx_row_stride, float* d_ln_w, float* d_ln_b, float* d_conv_w,
                       float* d_conv_b, void* ws, size_t ws_bytes, int64_t B, int64_t L, int64_t D,
                       float eps, int dtype, void* stream);

/*
 * Diagonal selective scan over ds channels.  For row (b,t) of projs, columns
 * [0,ds) hold dt_raw, [ds,2ds) x and [2ds,3ds) b.  With dt = softplus(dt_raw)
 * (threshold 20) and A = -exp(A_log): h_t = h_{t-1} * exp(dt*A) + dt*b*x,
 * y[b,t,:] = h_t.  h0 [B,ds] fp32 (NULL = zeros); h_final [B,ds] fp32 or NULL.
 * y rows may alias the first ds columns of the `combined` buffer.
 * row_stats (fp32, or NULL): for row r = b*L+t and 32-channel block c, the pair
 * (sum, sum of squares) of the y values stored in that block (as rounded) is written to
 * row_stats[2*(c*stats_part_stride + r)] and the next float; stats_part_stride (in pairs)
 * >= B*L.  These are partial statistics for hdcm_rowln_gemm_stats_fwd.
 * One launch; every input row is read once.  ws: hdcm_ssm_workspace_bytes(B, L, ds) bytes,
 * 256-byte aligned, zero-filled before the first call that uses it and passed again as the
 * previous call left it (the kernel keeps a call counter in it and never needs it cleared
 * again; a buffer sized for larger inputs serves smaller ones).  Calls that share a
 * workspace must not overlap (order them on one stream).
 * Replaces: _ssm_intra_v2 + _ssm_scan_v2 + _ssm_inter_v2 launches and the
 *           y_ssm copy into `combined` (hdcmamba/model.py:345-363, 294-295).
 */
size_t hdcm_ssm_workspace_bytes(int64_t B, int64_t L, int64_t ds);
int hdcm_ssm_fwd(const void* projs, int64_t proj_row_stride, const void* A_log,
                 const float* h0, void* y, int64_t y_row_stride, float* h_final,
                 float* row_stats, int64_t stats_part_stride, void* ws, size_t ws_bytes,
                 int64_t B, int64_t L, int64_t ds, int dtype, void* stream);

/*
 * hdcm_ssm_fwd without a workspace argument: the same kernels and results, with their
 * scratch in a fixed device array of HDCM_SSM_NOALLOC_SCRATCH_BYTES that the library holds on
 * each GPU it runs on until the process ends.  The call allocates nothing (no hipMalloc, no
 * allocating library routine), so it can be used where allocation is not possible.  Inputs
 * whose workspace (hdcm_ssm_workspace_bytes) would exceed that size return HDCM_ETOOBIG.
 * Every call on one GPU uses that GPU's array: calls that overlap on one GPU (concurrent
 * streams) race; calls ordered on one stream do not.
 * No counterpart in the reference; for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid allocation).
 */
#define HDCM_SSM_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)
int hdcm_ssm_fwd_noalloc(const void* projs, int64_t proj_row_stride, const void* A_log,
                         const float* h0, void* y, int64_t y_row_stride, float* h_final,
                         float* row_stats, int64_t stats_part_stride, int64_t B, int64_t L,
                         int64_t ds, int dtype, void* stream);

/*
 * Gradient of hdcm_ssm_fwd from a zero start state: given gy (the gradient of y) and h (the
 * forward's y), writes d dt_raw, d x, d b into columns [0, 3*ds) of dprojs (the dtype of
 * projs) and d A_log (fp32 [ds], summed in a fixed order).  The adjoint g_t = gy_t +
 * a_{t+1} g_{t+1} is scanned like the forward, rows in reverse.  ws:
 * hdcm_ssm_bwd_workspace_bytes(B, L, ds, dtype) bytes, 256-byte aligned.
 * No reference counterpart (the reference's scan kernels have no backward,
 * hdcmamba/model.py:175-233,340-384); the forward is that of model.py:175-233.
 */
size_t hdcm_ssm_bwd_workspace_bytes(int64_t B, int64_t L, int64_t ds, int dtype);
int hdcm_ssm_bwd(const void* projs, int64_t proj_row_stride, const void* A_log, const void* h,
                 int64_t h_row_stride, const void* gy, int64_t gy_row_stride, void* dprojs,
                 int64_t dprojs_row_stride, float* dA_log, void* ws, size_t ws_bytes, int64_t B,
                 int64_t L, int64_t ds, int dtype, void* stream);

/*
 * Slot memory (per-head decayed linear attention, feature map elu+1) in two
 * calls sharing one workspace.  q, k, v and gate are the column blocks
 * [q_col, q_col+dm), [+dm, +2dm), [+2dm, +3dm), [+3dm, +4dm) of projs; head h
 * owns columns h*hd..h*hd+hd-1 of each block, hd = dm/H.  gamma [H] is the
 * per-head decay.  With chunk size C the weight of (t, j<=t) is gamma^(t-j)
 * inside t's chunk and gamma^(t-j-1) across chunks.
 *
 * hdcm_slot_state_fwd computes the chunk-boundary state at the start of every
 * sequence segment into ws (S0 [B,H,hd,hd] fp32 = state before row 0, or NULL).
 * hdcm_slot_gate_fwd then produces, per (token, head), GroupNorm over hd
 * (gn_eps, affine gn_w/gn_b [dm]) times sigmoid(gate), written to columns
 * [out_col, out_col+dm) of `out`; S_final [B,H,hd,hd] fp32 (or NULL) receives
 * the state after row L-1 (L must then be a multiple of C).  row_stats (fp32, or
 * NULL): for row r = b*L+t and head h, the pair (sum, sum of squares) of the hd values
 * stored (as rounded) at row_stats[2*(h*stats_part_stride + r)] and the next float;
 * stats_part_stride (in pairs) >= B*L (partial statistics for hdcm_rowln_gemm_stats_fwd).
 * Needs hd a multiple of 16 up to 128, and L a multiple of C (any C >= 1: a C that
 * neither divides the row tile of 64 rows (bf16) / 32 rows (fp32) nor is a multiple of it
 * is walked in tiles confined to one chunk each).
 * Replaces: _slot_all_fused launch (hdcmamba/model.py:366-371, kernel
 *           model.py:236-272) and the slot part of _fused_gnorm_gate_cat_kernel
 *           (model.py:375-380, kernel model.py:274-293).
 */
size_t hdcm_slot_workspace_bytes(int64_t B, int64_t L, int64_t dm, int64_t H, int64_t C,
                                 int dtype);
int hdcm_slot_state_fwd(const void* projs, int64_t proj_row_stride, int64_t q_col,
                        const void* gamma, const float* S0, void* ws, size_t ws_bytes,
                        int64_t B, int64_t L, int64_t dm, int64_t H, int64_t C,
                        int dtype, void* stream);
int hdcm_slot_gate_fwd(const void* projs, int64_t proj_row_stride, int64_t q_col,
                       const void* gamma, const void* gn_w, const void* gn_b, float gn_eps,
                       const void* ws, size_t ws_bytes, void* out, int64_t out_row_stride,
                       int64_t out_col, float* S_final, float* row_stats, int64_t stats_part_stride,
                       int64_t B, int64_t L, int64_t dm, int64_t H, int64_t C, int dtype,
                       void* stream);

/*
 * The slot recurrence without the GroupNorm and gate, on any three column blocks of one
 * row buffer:  y_t = sum_{j<=t} w(t,j) (f(q_t).f(k_j)) v_j  per head, with w the slot
 * weights above, f = phi (phi != 0) or the identity, q/k/v at columns q_col/k_col/v_col
 * (+ h*hd) of `base`, y written to columns [out_col, out_col+dm) of `out`.  A negative
 * row stride runs the sequence backwards: `base` (or `out`) then points at the row of the
 * last token of the last batch and rows are reached at base + (b*L + t) * row_stride;
 * with L a multiple of C the chunk grid maps onto itself.  Same workspace as the slot
 * pair above (hdcm_slot_workspace_bytes).  The slot memory's backward runs it four times:
 * to recompute y (phi, forward) and for dphi(q) (identity: q=dy, k=v, v=phi(k)), dv
 * (backwards: q=phi(k), k=phi(q), v=dy) and dphi(k) (backwards: q=v, k=dy, v=phi(q)).
 * With `chain` non-NULL each output value is multiplied by phi'(z) = 1 (z > 0) else exp(z),
 * z read from `chain` at the output's own row and column (chain has out's column layout and
 * row stride chain_row_stride, negative with a negative out_row_stride): dphi(q) and dphi(k)
 * become dq and dk in the same pass.
 * No reference counterpart (the reference's slot kernel has no backward,
 * hdcmamba/model.py:236-272,340-384); the weights are those of model.py:265-272.
 */
int hdcm_slot_attend_fwd(const void* base, int64_t row_stride, int64_t q_col, int64_t k_col,
                         int64_t v_col, const void* gamma, int phi, void* ws, size_t ws_bytes,
                         void* out, int64_t out_row_stride, int64_t out_col, const void* chain,
                         int64_t chain_row_stride, int64_t B, int64_t L, int64_t dm, int64_t H,
                         int64_t C, int dtype, void* stream);

/*
 * The per-token, per-head GroupNorm (eps, affine gn_w/gn_b over hd = dm/H values) and sigmoid
 * gate of hdcm_slot_gate_fwd as a pass of its own, for heads wider than that pass holds
 * (hd > 128): out = GN(y) * sigmoid(gate) on `rows` token rows, y = y1 + y2', y2' being y2
 * with the two halves of every head exchanged (y2 may be NULL; with it hd must be even), so
 * that a head of 2*hb columns can run its slot recurrence as two sub-heads of hb through
 * hdcm_slot_attend_fwd (equal key and value blocks in y1, crossed ones in y2 after its value
 * halves were exchanged).  row_stats (or NULL): per row r and head h the (sum, sum of squares)
 * of the hd stored values at row_stats[2*(h*stats_part_stride + r)], as hdcm_slot_gate_fwd
 * writes them.  hd <= 512.
 * Replaces: the slot part of _fused_gnorm_gate_cat_kernel (hdcmamba/model.py:274-293, launch
 * model.py:375-380), whose BLOCK_SIZE_D = max(64, next_pow2(hd)) covers any head dim.
 */
int hdcm_gnorm_gate_fwd(const void* y1, int64_t y1_row_stride, const void* y2, int64_t y2_row_stride,
                        const void* gate, int64_t gate_row_stride, const void* gn_w, const void* gn_b, float gn_eps,
                        void* out, int64_t out_row_stride, float* row_stats, int64_t stats_part_stride,
                        int64_t rows, int64_t dm, int64_t H, int dtype, void* stream);

/*
 * Gradient of the per-token, per-head GroupNorm (eps, affine gn_w/gn_b over hd = dm/H
 * values) and sigmoid gate of hdcm_slot_gate_fwd, on `rows` token rows: from y (the slot
 * recurrence's output before the GroupNorm), the gate values and dout, writes dy and dgate
 * (activation dtype) and d gn_w, d gn_b (fp32 [dm], summed in a fixed order).
 * ws: hdcm_gnorm_gate_bwd_workspace_bytes(dm, H) bytes.  hd a multiple of 16 up to 128.
 * No reference counterpart (model.py:274-295 has no backward).
 */
size_t hdcm_gnorm_gate_bwd_workspace_bytes(int64_t dm, int64_t H);
int hdcm_gnorm_gate_bwd(const void* y, int64_t y_row_stride, const void* gate, int64_t gate_row_stride,
                        const void* gn_w, const void* gn_b, float eps, const void* dout,
                        int64_t dout_row_stride, void* dy, int64_t dy_row_stride, void* dgate,
                        int64_t dgate_row_stride, float* dgn_w, float* dgn_b, void* ws, size_t ws_bytes,
                        int64_t rows, int64_t dm, int64_t H, int dtype, void* stream);

/*
 * Operands of the slot recurrence's gradient passes.  hdcm_slot_phi_prep writes, per row,
 * v, phi(k) and phi(q) (rounded to the dtype) into column blocks [dm, 2dm), [2dm, 3dm) and
 * [3dm, 4dm) of z (q, k, v at columns q_col, +dm, +2dm of projs).  hdcm_slot_phi_chain turns
 * the gradients of phi(q), phi(k) held in the q and k column blocks of dprojs into those of
 * q, k in place: multiplied by phi'(z) = 1 for z > 0, exp(z) otherwise.
 * No reference counterpart (the feature map of model.py:261-262 has no backward).
 */
int hdcm_slot_phi_prep(const void* projs, int64_t proj_row_stride, int64_t q_col, void* z,
                       int64_t z_row_stride, int64_t rows, int64_t dm, int dtype, void* stream);
int hdcm_slot_phi_chain(const void* projs, int64_t proj_row_stride, int64_t q_col, void* dprojs,
                        int64_t dprojs_row_stride, int64_t rows, int64_t dm, int dtype, void* stream);

/*
 * Recurrent decode (one token per batch row) after a prefill.  No counterpart in the
 * reference, whose only generation path re-runs the whole forward
 * (hdcmamba/train.py:139-151); the semantics are those of the chunked forward continued
 * token by token (hdcmamba/model.py:22-72, 175-233, 236-295).
 *
 * hdcm_norm_conv_step_fwd: LayerNorm + causal width-4 conv of x[b,:] (row stride
 * x_row_stride) using hist [B,3,D] (activation dtype, contiguous), the raw block-input
 * rows t-3, t-2, t-1 (zero rows before the sequence start, whose LayerNorm is ln_b).
 * Writes out[b,:] and shifts x into hist.  Same weights as hdcm_norm_conv_fwd; needs
 * D % (16/elt_size) == 0 and D/(16/elt_size) <= 1024.
 *
 * hdcm_mixer_step_fwd: one token of the SSM (h [B,ds] fp32, updated) and of the slot
 * memory + GroupNorm + gate, reading one projs row per batch row (columns as in
 * hdcm_ssm_fwd at 0 and hdcm_slot_state_fwd at q_col).  The slot state is the pair
 * S_prev [B,H,hd,hd] (chunk-boundary state, as hdcm_slot_gate_fwd's S_final) and
 * S_intra [B,H,hd,hd] (between the tokens of a chunk: the last token's effective state,
 * its chunk's own decayed sum plus gamma^pos S_prev; not read at a chunk start), both fp32
 * and updated; pos = t mod C is the token's offset in its chunk (0 right after a prefill,
 * whose padded length is a multiple of C).  Writes y_ssm to columns [y_col, y_col+ds) and
 * the gated slot output to [g_col, g_col+dm) of out.  Needs hd a multiple of 16 up to 128 and
 * 16-byte aligned S_prev / S_intra.  With pos_dev
 * non-NULL the offset is read from that device int32 instead of pos, so one captured
 * graph of a decode step serves every position; hdcm_chunk_pos_advance then moves it to
 * (pos + 1) mod C on the stream (no counterpart in the reference: graph replay support).
 */
int hdcm_norm_conv_step_fwd(const void* x, int64_t x_row_stride, const void* ln_w,
                            const void* ln_b, const void* conv_w, const void* conv_b, void* hist,
                            void* out, int64_t out_row_stride, int64_t B, int64_t D, float eps,
                            int dtype, void* stream);
int hdcm_mixer_step_fwd(const void* projs, int64_t proj_row_stride, int64_t q_col,
                        const void* A_log, float* h, const void* gamma, float* S_prev,
                        float* S_intra, int64_t pos, const int32_t* pos_dev, int64_t C,
                        const void* gn_w, const void* gn_b, float gn_eps, void* out,
                        int64_t out_row_stride, int64_t y_col, int64_t g_col, int64_t B,
                        int64_t dm, int64_t ds, int64_t H, int dtype, void* stream);
int hdcm_chunk_pos_advance(int32_t* pos_dev, int64_t C, void* stream);

/*
 * Skinny bf16 GEMM of the decode step: out[m,n] = sum_k A[m,k] W[n,k] (+ bias[n])
 * (+ res[m,n]) for m < M <= 16, fp32 accumulation, one rounding to bf16.  W is an
 * nn.Linear weight [N,K] (row stride w_row_stride); bias [N] and res (row stride
 * res_row_stride) may be NULL; res may alias out.  Needs K % 32 == 0, K <= 3072 and
 * 16-byte aligned rows of A and W.
 * Replaces, in the decode step only, the nn.Linear projections in_proj and out_proj
 * (hdcmamba/model.py:313,325,340,383; the residual add of model.py:394) and the tied LM
 * head (train_fineweb.py:55,94).
 */
int hdcm_skinny_gemm_fwd(const void* A, int64_t a_row_stride, const void* W, int64_t w_row_stride,
                         const void* bias, const void* res, int64_t res_row_stride, void* out,
                         int64_t out_row_stride, int64_t M, int64_t N, int64_t K, int dtype,
                         void* stream);

/*
 * The front of a decode step in one launch: hdcm_norm_conv_step_fwd of x (B rows, D = K
 * columns; u = its output, hist shifted) followed by hdcm_skinny_gemm_fwd(u, W, bias) into
 * out [B,N] -- the same values, bit for bit, as those two calls.  The GEMM's weight loads are
 * issued while the conv rows are computed; its workgroups wait for the rows on flags in the
 * workspace (ws, at least hdcm_step_workspace_bytes() bytes, 128-byte aligned, zero-filled
 * before the first call and then kept by the caller for every later call; calls that overlap
 * on one workspace race).  The 32-bit word at byte 128 of the workspace counts waits that gave
 * up after HDCM_OPT_STEP_SPIN_ROUNDS polls (0 unless the GPU is shared with work that holds
 * back the conv rows' workgroups; outputs of such a call are not valid).  bf16 only;
 * 1 <= B <= 16, D % 32 == 0, D <= 2048; bias may be NULL.
 * Replaces: the block's norm + conv1d then in_proj of one token (hdcmamba/model.py:22-72
 * per row, then model.py:313,340); no counterpart as one call (the reference has no decode
 * step, hdcmamba/train.py:139-151).
 */
size_t hdcm_step_workspace_bytes(void);
int hdcm_norm_conv_in_proj_step_fwd(const void* x, int64_t x_row_stride, const void* ln_w, const void* ln_b,
                                    const void* conv_w, const void* conv_b, void* hist, float eps, void* u,
                                    int64_t u_row_stride, const void* W, int64_t w_row_stride,
                                    const void* bias, void* out, int64_t out_row_stride, int64_t B,
                                    int64_t D, int64_t N, void* ws, size_t ws_bytes, int dtype,
                                    void* stream);

/*
 * Tiled bf16 GEMM: out[t,o] = sum_k x[t,k] w[o,k] (+ bias[o]) for t < M, o < N, fp32
 * accumulation, one rounding to bf16.  w is an nn.Linear weight [N,K]; bias may be NULL.
 * Needs K % 8 == 0, N % 4 == 0, 16-byte aligned rows of x and w, 8-byte aligned out.
 * Replaces the nn.Linear in_proj of the prefill/forward (hdcmamba/model.py:313,340).
 */
int hdcm_gemm_fwd(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride,
                  const void* bias, void* out, int64_t out_row_stride, int64_t M, int64_t N, int64_t K,
                  int dtype, void* stream);

/*
 * out_proj over the row LayerNorm without affine, with the residual add:
 *   out[t,o] = res[t,o] + r_t * (sum_k c[t,k] w[o,k] - mu_t * s_o),  s_o = sum_k w[o,k]
 * which equals res + LN(c) w^T with LN(c)_t = (c_t - mu_t) r_t over the K columns of row t
 * (mu_t the mean, r_t = 1/sqrt(var_t + eps), biased variance).  mu, r and s are computed in
 * the kernel from the operands it multiplies.  res may alias out.  Alignment as
 * hdcm_gemm_fwd.  Replaces F.layer_norm(combined.float(), (ds+dm,)).to(dtype), out_proj and
 * the residual add (hdcmamba/model.py:382-383,394).
 */
int hdcm_rowln_gemm_fwd(const void* c, int64_t c_row_stride, const void* w, int64_t w_row_stride,
                        const void* res, int64_t res_row_stride, void* out, int64_t out_row_stride,
                        int64_t M, int64_t N, int64_t K, float eps, int dtype, void* stream);

/*
 * hdcm_rowln_gemm_fwd with mu, r and s supplied instead of computed: row_stats holds, per
 * row t of c, stats_parts pairs (sum, sum of squares) of disjoint column blocks that cover
 * the K columns, pair p of row t at row_stats[2*(p*stats_part_stride + t)] (as
 * hdcm_ssm_fwd and hdcm_slot_gate_fwd write them when given the same buffer), summed in
 * order of p; w_sums [N] fp32 = hdcm_row_sums_fwd of w.  Same result up to
 * fp32 summation order.  Needs N, res_row_stride and out_row_stride multiples of 8 and res,
 * out and w_sums 16-byte aligned.  res may alias out.  Replaces, like hdcm_rowln_gemm_fwd,
 * F.layer_norm(combined.float(), (ds+dm,)).to(dtype), out_proj and the residual add
 * (hdcmamba/model.py:382-383,394).
 */
int hdcm_rowln_gemm_stats_fwd(const void* c, int64_t c_row_stride, const void* w, int64_t w_row_stride,
                              const float* w_sums, const float* row_stats, int64_t stats_parts,
                              int64_t stats_part_stride, const void* res, int64_t res_row_stride, void* out, int64_t out_row_stride,
                              int64_t M, int64_t N, int64_t K, float eps, int dtype, void* stream);

/*
 * sums[o] = sum_k w[o, k] in fp32 over the K columns of each of N bf16 rows: the weight
 * row sums hdcm_rowln_gemm_stats_fwd takes (computed once per weight).  No reference
 * counterpart; part of the out_proj fold above.
 */
int hdcm_row_sums_fwd(const void* w, int64_t w_row_stride, int64_t N, int64_t K, float* sums, int dtype,
                      void* stream);

/*
 * Row LayerNorm over `width` columns, fp32 statistics, optional affine
 * (w, b may be NULL).  in and out may be the same buffer.
 * Replaces: F.layer_norm(combined.float(), (ds+dm,)).to(dtype)
 *           (hdcmamba/model.py:382) and norm_final (model.py:400,404).
 */
int hdcm_rowln_fwd(const void* in, int64_t in_row_stride, void* out, int64_t out_row_stride,
                   const void* w, const void* b, int64_t rows, int64_t width, float eps,
                   int dtype, void* stream);

/*
 * Two affine row LayerNorms in one pass: out = LN(LN(in; w1, b1, eps1); w2, b2, eps2), the
 * intermediate rounded to the activation dtype as a stored tensor is, by the same per-row
 * code as hdcm_rowln_fwd, so the result equals two hdcm_rowln_fwd calls bit for bit.
 * in and out may be the same buffer.  width up to 512 16-byte groups (4096 bf16 or 2048 fp32
 * columns), HDCM_EUNSUPPORTED beyond.
 * Replaces: norm_final (hdcmamba/model.py:400,404) followed by the LM wrapper's norm_f
 *           (train_fineweb.py:67,94) in the LM forward.
 */
int hdcm_rowln2_fwd(const void* in, int64_t in_row_stride, void* out, int64_t out_row_stride,
                    const void* w1, const void* b1, float eps1, const void* w2, const void* b2, float eps2,
                    int64_t rows, int64_t width, int dtype, void* stream);

/*
 * Gradient of hdcm_rowln_fwd: dx (x's dtype) from dy and the forward input x (the row
 * statistics are recomputed in fp32); with affine (w non-NULL) also dw = sum_rows dy*x^ and
 * db = sum_rows dy as fp32 [width], summed in a fixed order (ws: per-workgroup partials,
 * hdcm_rowln_bwd_workspace_bytes(rows, width) bytes; unused without affine).
 * width/E <= 512 (E = 8 bf16, 4 fp32 elements per 16 bytes).
 * Replaces: the autograd backward of nn.LayerNorm / F.layer_norm for norm_final
 *           (hdcmamba/model.py:400,404), the LM's norm_f (train_fineweb.py:52,92) and the
 *           post-LayerNorm (model.py:382).
 */
size_t hdcm_rowln_bwd_workspace_bytes(int64_t rows, int64_t width);
int hdcm_rowln_bwd(const void* dy, int64_t dy_row_stride, const void* x, int64_t x_row_stride,
                   const void* w, void* dx, int64_t dx_row_stride, float* dw, float* db, void* ws,
                   size_t ws_bytes, int64_t rows, int64_t width, float eps, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HDCM_H_ */
