"""HdcMamba block and model on MI355X: the reference module surface over HIP kernels.

Drop-in for hdcmamba/model.py of N01N9/hdcmamba: the class and function names,
constructor signatures, parameter/buffer names and shapes, and the order in which
construction consumes the global RNG (so ``torch.manual_seed(s)`` followed by
construction yields the same weights) are those of the reference.  The forward of a
block runs, per layer:

    norm_conv (HIP)  ->  in_proj (hipBLASLt GEMM)  ->  ssm (HIP) and slot state, scan and
    gate (HIP) writing one `combined` row buffer
    ->  bf16 without autograd: one HIP GEMM applying the row LayerNorm of `combined` in its
        epilogue (row statistics handed over by the ssm and gate kernels), out_proj and the
        residual add, in place on the residual stream;
        otherwise: row LayerNorm (HIP, in place) -> out_proj with the residual (addmm)

Intended semantics are computed (see the oracle's docstring for the reference kernel
defects that are not reproduced).  Only GPU tensors are accepted; there is no CPU path.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

from . import _ops

__all__ = ["HdcMamba9v3Block", "HdcMamba9v3Model", "FusedNormConv1dFunction",
           "fused_norm_conv1d_trainable", "RowLayerNormFunction", "layer_norm", "SlotSsmMixerFunction",
           "set_differentiable_mixer", "set_fused_out_proj", "set_fused_step_front", "BlockState"]


@dataclass
class BlockState:
    """What one block carries from a prefill into single-token steps.

    conv     [B,3,dm]     block-input rows t-3..t-1 (activation dtype; zero rows before the
                          sequence start, whose LayerNorm is the LayerNorm bias)
    h        [B,ds]       SSM state, fp32
    S_prev   [B,H,hd,hd]  slot state at the last chunk boundary, fp32
    S_intra  [B,H,hd,hd]  between the tokens of a chunk, the last token's effective slot
                          state (the chunk's own decayed sum plus gamma^c S_prev), fp32;
                          not read at a chunk start
    pos                   offset of the next token inside its chunk
    """
    conv: torch.Tensor
    h: torch.Tensor
    S_prev: torch.Tensor
    S_intra: torch.Tensor
    pos: int = 0


class FusedNormConv1dFunction(torch.autograd.Function):
    """LayerNorm + causal depthwise conv1d (width 4) on the HIP kernels.

    Same ``apply(x, norm_weight, norm_bias, conv_weight[D,4], conv_bias, eps)`` signature
    and backward outputs (dx and the four parameter gradients in x's dtype, None for eps)
    as hdcmamba/model.py:126-166.  The backward is the exact gradient of the forward,
    including the LayerNorm bias terms (also through the LayerNorm of the zero rows before
    the sequence start) that the reference's backward kernel leaves out, from fp32 row
    statistics.
    """

    @staticmethod
    def forward(ctx, x, norm_weight, norm_bias, conv_weight, conv_bias, eps):
        ctx.save_for_backward(x, norm_weight, norm_bias, conv_weight)
        ctx.eps = eps
        return _ops.norm_conv(x, norm_weight, norm_bias, conv_weight, conv_bias, eps)

    @staticmethod
    def backward(ctx, grad_output):
        x, norm_weight, norm_bias, conv_weight = ctx.saved_tensors
        dx, dnw, dnb, dcw, dcb = _ops.norm_conv_bwd(grad_output, x, norm_weight, norm_bias, conv_weight, ctx.eps)
        return (dx, dnw.to(x.dtype), dnb.to(x.dtype), dcw.to(x.dtype).view_as(conv_weight), dcb.to(x.dtype),
                None)


def fused_norm_conv1d_trainable(x, norm_layer, conv_layer):
    """hdcmamba/model.py:168-172: weights cast to x.dtype, conv weight squeezed to [D,4]."""
    return FusedNormConv1dFunction.apply(
        x, norm_layer.weight.to(x.dtype), norm_layer.bias.to(x.dtype),
        conv_layer.weight.squeeze(1).to(x.dtype), conv_layer.bias.to(x.dtype), norm_layer.eps)


class RowLayerNormFunction(torch.autograd.Function):
    """LayerNorm over the last dim on the HIP kernels, forward and backward, with the
    semantics of nn.LayerNorm / F.layer_norm (fp32 statistics, output in x's dtype).

    ``apply(x, weight, bias, eps)``; weight and bias may both be None (no affine).  The
    parameter gradients are summed over rows in fp32 in a fixed order and returned in the
    parameters' dtype.
    """

    @staticmethod
    def forward(ctx, x, weight, bias, eps):
        ctx.eps = float(eps)
        ctx.w_dtype = weight.dtype if weight is not None else None
        ctx.save_for_backward(x, weight)
        return _ops.layer_norm(x.contiguous(), weight, bias, eps)

    @staticmethod
    def backward(ctx, grad_out):
        x, weight = ctx.saved_tensors
        dx, dw, db = _ops.layer_norm_bwd(grad_out.to(x.dtype), x.contiguous(), weight, ctx.eps)
        if weight is None:
            return dx, None, None, None
        return dx, dw.to(ctx.w_dtype), db.to(ctx.w_dtype), None


def layer_norm(x, weight=None, bias=None, eps=1e-5):
    """Row LayerNorm on the HIP kernels; goes through RowLayerNormFunction when autograd
    needs its gradient (training the residual path, norm_final and the LM's norm_f)."""
    needs = torch.is_grad_enabled() and (x.requires_grad or any(
        t is not None and t.requires_grad for t in (weight, bias)))
    if needs:
        return RowLayerNormFunction.apply(x, weight, bias, eps)
    return _ops.layer_norm(x.contiguous(), weight, bias, eps)


class SlotSsmMixerFunction(torch.autograd.Function):
    """The block's SSM and slot memory + GroupNorm/gate on the HIP kernels, differentiable.

    ``apply(projs, A_log, gamma, gn_w, gn_b, d_state, d_model, num_heads, chunk)`` returns
    the ``combined`` rows [y_ssm | gated slot output] of the forward (model.py:345-380).
    The backward (no counterpart in the reference, whose kernels have no autograd) returns
    the gradients of projs, A_log and the GroupNorm parameters; gamma (the slot decay, a
    buffer refreshed from decay_log) is treated as a constant.  Slot part: y recomputed by
    the plain recurrence, the GroupNorm/gate backward, then three passes of the recurrence
    for d phi(q), d v and d phi(k) (the last two backwards in time) and the phi' chain;
    SSM part: the adjoint scan from the forward's y.
    """

    @staticmethod
    def forward(ctx, projs, A_log, gamma, gn_w, gn_b, ds, dm, H, C):
        B, L, _ = projs.shape
        combined = torch.empty(B, L, ds + dm, device=projs.device, dtype=projs.dtype)
        _ops.ssm(projs, A_log, ds, combined[..., :ds])
        ws = _ops.slot_workspace(projs, dm, H, C)
        _ops.slot_state(projs, 3 * ds, gamma, dm, H, C, ws)
        _ops.slot_gate(projs, 3 * ds, gamma, gn_w, gn_b, 1e-5, ws, combined, ds, dm, H, C)
        ctx.save_for_backward(projs, A_log, gamma, gn_w, gn_b, combined)
        ctx.dims = (ds, dm, H, C)
        return combined

    @staticmethod
    def backward(ctx, dcomb):
        projs, A_log, gamma, gn_w, gn_b, combined = ctx.saved_tensors
        ds, dm, H, C = ctx.dims
        B, L, _ = projs.shape
        dcomb = dcomb.to(projs.dtype).contiguous()
        q_col, g_col = 3 * ds, 3 * ds + 3 * dm
        dprojs = torch.empty_like(projs)
        ws = _ops.slot_workspace(projs, dm, H, C)
        y = torch.empty(B, L, dm, device=projs.device, dtype=projs.dtype)
        _ops.slot_attend(projs, q_col, q_col + dm, q_col + 2 * dm, gamma, dm, H, C, True, y, 0, ws=ws)
        z = torch.empty(B, L, 4 * dm, device=projs.device, dtype=projs.dtype)  # [dy | v | phi(k) | phi(q)]
        dgw, dgb = _ops.gnorm_gate_bwd(y, projs[..., g_col:], gn_w, gn_b, 1e-5, dcomb[..., ds:], H,
                                       z[..., :dm], dprojs[..., g_col:])
        _ops.slot_phi_prep(projs, q_col, dm, z)
        # d q = d phi(q) * phi'(q) and d k likewise: the passes multiply by phi' of the
        # projections (chain) as they store
        _ops.slot_attend(z, 0, dm, 2 * dm, gamma, dm, H, C, False, dprojs, q_col, ws=ws, chain=projs)  # d q
        _ops.slot_attend(z, 2 * dm, 3 * dm, 0, gamma, dm, H, C, False, dprojs, q_col + 2 * dm, reverse=True,
                         ws=ws)  # d v
        _ops.slot_attend(z, dm, 0, 3 * dm, gamma, dm, H, C, False, dprojs, q_col + dm, reverse=True,
                         ws=ws, chain=projs)  # d k
        dA = _ops.ssm_bwd(projs, A_log, ds, combined[..., :ds], dcomb[..., :ds], dprojs)
        return (dprojs, dA.to(A_log.dtype), None, dgw.to(gn_w.dtype), dgb.to(gn_b.dtype), None, None, None, None)


class HdcMamba9v3Block(nn.Module):
    """SSM + slot-memory block (hdcmamba/model.py:300-394).

    ``forward(x[B,L,d_model]) -> (y[B,L,d_model], None)``.  L is left-padded with zero
    rows to a multiple of ``chunk_size`` and the pad is sliced off the output
    (model.py:388-389,394).

    As in the reference, backward reaches out_proj and the residual only: the SSM and slot
    kernels are constants for autograd.  With ``differentiable_mixer = True`` (an added
    option) the training forward runs them through SlotSsmMixerFunction instead, so
    in_proj, the LN+conv, A_log and the GroupNorm receive gradients too.

    ``fused_out_proj`` (added, on by default): without autograd and in bf16, the LayerNorm
    of `combined`, out_proj and the residual add run as one GEMM whose epilogue applies the
    LayerNorm (hdcm_rowln_gemm_fwd) at the shapes where that measured faster (see
    ``_fused_out``); otherwise as a row LayerNorm kernel and addmm.
    """

    # where the SSM's launch overlaps the slot kernels (see _mixer): "auto" runs it in sequence
    # while a HIP graph is being recorded and beside the slot pre-pass and scan otherwise.
    # Measured at the 24-layer d_model=1024 L=32768 forward: recorded graph 14.46 ms per
    # forward in sequence against 14.59 overlapped (with no launch gaps to fill, the scan's
    # workgroups only slow the pre-pass: 25 + 55 us against 24 + 28 us); eager forwards 15.14
    # overlapped against 15.65 in sequence.
    ssm_overlap = "auto"
    # decode step: the LayerNorm + conv of the token and in_proj as one launch
    # (hdcm_norm_conv_in_proj_step_fwd: in_proj's weight stream starts while the conv rows are
    # computed; the same values as the two kernels) where in_proj runs on the wide skinny GEMM
    # (at least 2048 outputs, d_model <= 2048); set_fused_step_front switches it.
    fused_step_front = True

    def __init__(self, d_model=512, d_state=64, num_heads=8, chunk_size=256, differentiable_mixer=False,
                 fused_out_proj=True):
        super().__init__()
        self.differentiable_mixer = differentiable_mixer
        self.fused_out_proj = fused_out_proj
        self.d_model, self.d_state = d_model, d_state
        self.num_heads, self.chunk_size = num_heads, chunk_size
        self.head_dim = d_model // num_heads
        proj = 3 * d_state + 4 * d_model

        # Construction order fixes the RNG stream (model.py:306-327).
        self.norm = nn.LayerNorm(d_model)
        self.conv1d = nn.Conv1d(d_model, d_model, kernel_size=4, groups=d_model, padding=3, bias=True)
        with torch.no_grad():
            nn.init.normal_(self.conv1d.weight, std=0.02)
            self.conv1d.weight[:, 0, -1] += 1.0  # start close to the identity tap
            self.conv1d.bias.zero_()
        self.in_proj = nn.Linear(d_model, proj, bias=True)
        with torch.no_grad():
            lo, hi = 0.001, 0.1  # dt = softplus(bias) starts uniform in [lo, hi]
            dt0 = torch.rand(d_state) * (hi - lo) + lo
            self.in_proj.bias[:d_state] = torch.log(torch.exp(dt0) - 1.0)
            q0, gate0 = 3 * d_state, 3 * d_state + 3 * d_model
            nn.init.xavier_uniform_(self.in_proj.weight[q0:gate0])
            self.in_proj.bias[gate0:].fill_(1.0)
        self.A_log = nn.Parameter(torch.log(torch.linspace(0.99, 0.9999, d_state)))
        self.decay_log = nn.Parameter(torch.log(torch.full((num_heads,), 0.05)))
        self.out_proj = nn.Linear(d_state + d_model, d_model, bias=False)
        self.group_norm = nn.GroupNorm(num_heads, d_model)
        self.register_buffer("gamma_buf", torch.exp(-F.softplus(self.decay_log)))

    def _mixer(self, x, state=None, normalize=True, row_stats=None):
        """LN+conv, in_proj, SSM and slot+gate into one `combined` row buffer, then (with
        ``normalize``) its LayerNorm in place (model.py:338-382).  x: chunk-aligned [B,L,dm].
        With ``state``, the SSM and slot states after the last row are written into it.  With
        ``row_stats`` ([P, B*L, 2] fp32) the SSM and the gate also write each row's partial
        (sum, sum of squares): the SSM's 32-channel blocks first, then one part per head."""
        B, L, dm = x.shape
        ds, H, C = self.d_state, self.num_heads, self.chunk_size
        dtype = x.dtype
        x_conv = fused_norm_conv1d_trainable(x, self.norm, self.conv1d)
        projs = F.linear(x_conv, self.in_proj.weight.to(dtype), self.in_proj.bias.to(dtype))
        combined = torch.empty(B, L, ds + dm, device=x.device, dtype=dtype)
        # The SSM and the slot kernels read projs and write disjoint columns of `combined`,
        # so the SSM may run on a side stream beside some of the slot kernels (ssm_overlap:
        # "state" = beside the state pre-pass and scan, "after_state" = beside the scan and
        # the gate pass, "gate" = beside all three, "none" = before them, the main stream
        # waiting for it; "auto" = "none" under graph capture, else "state").  The
        # join before the return orders every later use (and the allocator's reuse) of projs
        # and combined after the SSM.
        main = torch.cuda.current_stream(x.device)
        mode = self.ssm_overlap
        if mode == "auto":
            mode = "none" if torch.cuda.is_current_stream_capturing() else "state"
        side = _ops.side_stream(x.device)  # one stream per device: the scan's workspace is kept per stream

        def run_ssm():
            side.wait_stream(main)
            with torch.cuda.stream(side):
                _ops.ssm(projs, self.A_log, ds, combined[..., :ds], h_final=None if state is None else state.h,
                         row_stats=row_stats, stats_part=0)
            if mode == "none":
                main.wait_stream(side)

        gamma = self.gamma_buf.to(dtype)
        q_col = 3 * ds
        if self.head_dim > _ops.SLOT_MAX_HEAD_DIM:
            mode = "none"  # the scan first (run_ssm reads mode when called)
            run_ssm()
            self._wide_slot_gate(projs, combined, gamma, row_stats, state)
            if normalize:
                _ops.layer_norm(combined, eps=1e-5, out=combined)
            return combined.view(B * L, ds + dm)
        ws = _ops.slot_workspace(projs, dm, H, C)
        if mode != "after_state":
            run_ssm()
        _ops.slot_state(projs, q_col, gamma, dm, H, C, ws)
        if mode == "after_state":
            run_ssm()
        if mode == "state":
            main.wait_stream(side)
        _ops.slot_gate(projs, q_col, gamma, self.group_norm.weight, self.group_norm.bias, 1e-5, ws,
                       combined, ds, dm, H, C, S_final=None if state is None else state.S_prev,
                       row_stats=row_stats, stats_part=_ops.ssm_stats_parts(ds))
        if mode in ("gate", "after_state"):
            main.wait_stream(side)
        if normalize:
            _ops.layer_norm(combined, eps=1e-5, out=combined)
        return combined.view(B * L, ds + dm)

    def _wide_slot_gate(self, projs, combined, gamma, row_stats, state):
        """Slot memory + GroupNorm + gate for a head dim above the fused kernels' 128 (the
        reference pads any head dim, model.py:245-246,286): a head of hd = 2 hb columns runs as two
        sub-heads of hb through the plain slot pass (hdcm_slot_attend_fwd, the head's decay for
        both).  The scores split over the two key blocks, phi(q).phi(k) = sum_b phi(q_b).phi(k_b),
        so value block c of the output is attend(q_c, k_c, v_c) + attend(q_b, k_b, v_c), b != c: the
        first pass gives the equal-block terms, the second, after the two value halves of every
        head in projs are exchanged, the crossed ones (at the other half's columns); then the
        GroupNorm over all hd values of their sum and the gate (hdcm_gnorm_gate_fwd).  projs'
        value columns are left exchanged.  Forward only: hd a multiple of 32 up to 256, no state
        hand-off."""
        B, L, _ = projs.shape
        dm, ds, H, C = self.d_model, self.d_state, self.num_heads, self.chunk_size
        hd = dm // H
        if hd % 32 or hd > 2 * _ops.SLOT_MAX_HEAD_DIM:
            raise _ops.HdcmError(f"slot memory (head dim {hd})", -3)
        if state is not None:
            raise _ops.HdcmError(f"slot memory state hand-off (head dim {hd})", -3)
        q_col = 3 * ds
        g2 = gamma.repeat_interleave(2)
        ws = _ops.slot_workspace(projs, dm, 2 * H, C)
        y1 = torch.empty(B, L, dm, device=projs.device, dtype=projs.dtype)
        y2 = torch.empty_like(y1)
        _ops.slot_attend(projs, q_col, q_col + dm, q_col + 2 * dm, g2, dm, 2 * H, C, True, y1, 0, ws=ws)
        v = projs[..., q_col + 2 * dm:q_col + 3 * dm].unflatten(-1, (H, 2, hd // 2))
        v.copy_(v.flip(-2))
        _ops.slot_attend(projs, q_col, q_col + dm, q_col + 2 * dm, g2, dm, 2 * H, C, True, y2, 0, ws=ws)
        _ops.gnorm_gate(y1, y2, projs[..., q_col + 3 * dm:], self.group_norm.weight, self.group_norm.bias, 1e-5, H,
                        combined[..., ds:], row_stats=row_stats, stats_part=_ops.ssm_stats_parts(ds))

    def _fused_out(self, x):
        """Whether out_proj runs as the GEMM with the LayerNorm folded in (bf16, no autograd).
        Measured: it pays on the decode step (<= 16 rows: the weight-streaming kernels) and
        up to ~1024 output tiles of 256 x 256 (the 32768-token d_model=1024 forward: 512);
        at the 131072-token d_model=2048 prefill (4096 tiles) hipBLASLt's out_proj plus the
        LayerNorm kernel is ~5 % faster than the tiled GEMM, so that shape keeps them."""
        if not (self.fused_out_proj and x.dtype == torch.bfloat16 and not torch.is_grad_enabled()
                and (self.d_state + self.d_model) % 8 == 0 and self.d_model % 4 == 0):
            return False
        rows = x.numel() // self.d_model
        tiles = -(-rows // 256) * -(-self.d_model // 256)
        return rows <= 16 or tiles <= 1024

    def _out_weight_sums(self, w):
        """Row sums of the out_proj weight as used (``w``, the activation-dtype weight), kept
        until the parameter changes (its storage or its version counter).  A refresh writes
        into the same buffer, so a recorded graph that reads it sees the new sums."""
        p = self.out_proj.weight
        key = (p.data_ptr(), p._version, w.dtype, w.device)
        if getattr(self, "_wsum_key", None) != key:
            old = getattr(self, "_wsum", None)
            if old is not None and old.device == w.device and old.numel() == w.shape[0]:
                _ops.row_sums(w, out=old)
            else:
                self._wsum = _ops.row_sums(w)
            self._wsum_key = key
        return self._wsum

    def refresh_derived_weights(self):
        """Bring the kept out_proj row sums up to date with the weight (a recorded forward
        graph calls this before each replay; it launches nothing when the weight is
        unchanged)."""
        if getattr(self, "_wsum_key", None) is None:
            return
        p = self.out_proj.weight
        if (p.data_ptr(), p._version) != self._wsum_key[:2]:
            self._out_weight_sums(p.to(self._wsum_key[2]))

    def _fused_mixer_out(self, x, state, out=None):
        """x + out_proj(LN(combined)) for the fused path, x [B,L,dm]; into ``out`` (which may be
        x) when given.  With more rows than a decode step the SSM and gate kernels hand the
        row statistics to the GEMM (hdcm_rowln_gemm_stats_fwd); otherwise the GEMM takes them
        from its operands (hdcm_rowln_gemm_fwd)."""
        B, L, dm = x.shape
        w = self.out_proj.weight.to(x.dtype)
        x2 = x.reshape(B * L, dm)
        o2 = None if out is None else out.view(B * L, dm)
        if _ops.rowln_stats_ok(x2, dm):
            parts = _ops.ssm_stats_parts(self.d_state) + self.num_heads
            stats = torch.empty(parts, B * L, 2, device=x.device, dtype=torch.float32)
            c = self._mixer(x, state, normalize=False, row_stats=stats)
            y = _ops.rowln_gemm_stats(c, w, self._out_weight_sums(w), stats, x2, out=o2)
        else:
            c = self._mixer(x, state, normalize=False)
            y = _ops.rowln_gemm(c, w, x2, out=o2)
        return y.view(B, L, dm)

    def _differentiable_mixer(self, x):
        """_mixer with autograd through every stage (differentiable_mixer)."""
        B, L, dm = x.shape
        ds, H, C = self.d_state, self.num_heads, self.chunk_size
        dtype = x.dtype
        x_conv = fused_norm_conv1d_trainable(x, self.norm, self.conv1d)
        projs = F.linear(x_conv, self.in_proj.weight.to(dtype), self.in_proj.bias.to(dtype))
        # gamma is a constant here (the buffer may carry its construction graph, as in the
        # reference's register_buffer of exp(-softplus(decay_log)))
        combined = SlotSsmMixerFunction.apply(projs, self.A_log.to(dtype), self.gamma_buf.detach().to(dtype),
                                              self.group_norm.weight.to(dtype), self.group_norm.bias.to(dtype),
                                              ds, dm, H, C)
        return layer_norm(combined, eps=1e-5).view(B * L, ds + dm)

    def _inner_forward(self, x, state=None):
        """Block body on a chunk-aligned [B,L,dm] input; returns x + out_proj(LN(combined))."""
        B, L, dm = x.shape
        if self._fused_out(x):
            return self._fused_mixer_out(x, state)
        if self.differentiable_mixer and state is None and torch.is_grad_enabled():
            if self.head_dim > _ops.SLOT_MAX_HEAD_DIM:
                raise _ops.HdcmError(f"differentiable slot memory (head dim {self.head_dim})", -3)
            c = self._differentiable_mixer(x)
        else:
            c = self._mixer(x, state)
        out = torch.addmm(x.reshape(B * L, dm), c, self.out_proj.weight.to(x.dtype).t())
        return out.view(B, L, dm)

    def _residual_step_(self, r, state=None):
        """In-place variant for a model-owned residual stream r [B,L,dm] (chunk-aligned):
        r += out_proj(LN(combined)), with the GEMM accumulating straight into r."""
        B, L, dm = r.shape
        if state is not None:
            self._capture_conv(r, state)
        if self._fused_out(r):
            self._fused_mixer_out(r, state, out=r)
            return r
        c = self._mixer(r, state)
        r.view(B * L, dm).addmm_(c, self.out_proj.weight.to(r.dtype).t())
        return r

    # ------------------------------------------------------------------ prefill / decode
    def new_state(self, batch, device, dtype):
        """The state before any token (what a prefill of an empty sequence leaves)."""
        dm, ds, H, hd = self.d_model, self.d_state, self.num_heads, self.head_dim
        return BlockState(conv=torch.zeros(batch, 3, dm, device=device, dtype=dtype),
                          h=torch.zeros(batch, ds, device=device),
                          S_prev=torch.zeros(batch, H, hd, hd, device=device),
                          S_intra=torch.zeros(batch, H, hd, hd, device=device), pos=0)

    @staticmethod
    def _capture_conv(xp, state):
        n = min(3, xp.shape[1])
        state.conv.zero_()
        state.conv[:, 3 - n:].copy_(xp[:, xp.shape[1] - n:])
        state.S_intra.zero_()
        state.pos = 0

    def prefill(self, x):
        """Forward over x [B,L,dm] that also returns the BlockState after its last token.
        The padded length is a multiple of the chunk, so the next token starts a chunk."""
        _ops._on_gpu(x)
        B, L_in, _ = x.shape
        pad = (self.chunk_size - (L_in % self.chunk_size)) % self.chunk_size
        xp = F.pad(x, (0, 0, pad, 0)).contiguous() if pad else x.contiguous()
        state = self.new_state(B, x.device, x.dtype)
        self._capture_conv(xp, state)
        y = self._inner_forward(xp, state)
        return y[:, pad:, :], state

    def step(self, x, state, pos_dev=None):
        """One token per batch row: x [B,dm] -> y [B,dm]; ``state`` advances in place.
        With ``pos_dev`` (int32 device scalar) the chunk offset is read on the device and
        state.pos is left to the caller (graph replay)."""
        _ops._on_gpu(x)
        dm, ds, H, C = self.d_model, self.d_state, self.num_heads, self.chunk_size
        B = x.shape[0]
        dtype = x.dtype
        w_in, b_in = self.in_proj.weight.to(dtype), self.in_proj.bias.to(dtype)
        conv_w = self.conv1d.weight.squeeze(1)
        if self.fused_step_front and w_in.shape[0] >= 2048 and _ops.norm_conv_in_proj_step_ok(x, w_in):
            _, projs = _ops.norm_conv_in_proj_step(x, self.norm.weight, self.norm.bias, conv_w, self.conv1d.bias,
                                                   self.norm.eps, state.conv, w_in, b_in)
        else:
            xc = _ops.norm_conv_step(x, self.norm.weight, self.norm.bias, conv_w, self.conv1d.bias, self.norm.eps,
                                     state.conv)
            # few rows: the weight-streaming skinny GEMM; otherwise the library GEMM
            projs = _ops.skinny_linear(xc, w_in, b_in) if _ops.skinny_ok(xc, w_in) else F.linear(xc, w_in, b_in)
        combined = torch.empty(B, ds + dm, device=x.device, dtype=dtype)
        _ops.mixer_step(projs, self.A_log, ds, 3 * ds, self.gamma_buf.to(dtype), self.group_norm.weight,
                        self.group_norm.bias, 1e-5, state.h, state.S_prev, state.S_intra, state.pos, C,
                        combined, dm, H, pos_dev=pos_dev)
        w_out = self.out_proj.weight.to(dtype)
        if self._fused_out(x):  # LayerNorm folded into the (skinny) out_proj GEMM
            y = _ops.rowln_gemm(combined, w_out, x)
        else:
            _ops.layer_norm(combined, eps=1e-5, out=combined)
            if _ops.skinny_ok(combined, w_out):
                y = _ops.skinny_linear(combined, w_out, residual=x)
            else:
                y = torch.addmm(x, combined, w_out.t())
        if pos_dev is None:
            state.pos = (state.pos + 1) % C
        return y

    def forward(self, x):
        _ops._on_gpu(x)
        B, L_in, _ = x.shape
        pad = (self.chunk_size - (L_in % self.chunk_size)) % self.chunk_size
        if pad > 0:
            x = F.pad(x, (0, 0, pad, 0))
        if self.training:
            with torch.no_grad():
                self.gamma_buf.copy_(torch.exp(-F.softplus(self.decay_log)))
            # the reference checkpoints the block body in training (model.py:391-392): only
            # x is kept for backward and the body runs again when the gradient is needed
            y = checkpoint(self._inner_forward, x.contiguous(), use_reentrant=False)
        else:
            y = self._inner_forward(x.contiguous())
        return y[:, pad:, :], None


class HdcMamba9v3Model(nn.Module):
    """Stack of blocks plus a final LayerNorm (hdcmamba/model.py:396-404).

    ``num_slots`` is accepted and unused, as in the reference.  ``chunk_size`` is an
    added keyword; its default 256 is the value the reference hard-codes.
    """

    def __init__(self, d_model, n_layers, d_state, num_slots, num_heads=8, chunk_size=256):
        super().__init__()
        self.layers = nn.ModuleList([
            HdcMamba9v3Block(d_model=d_model, d_state=d_state, num_heads=num_heads, chunk_size=chunk_size)
            for _ in range(n_layers)])
        self.norm_final = nn.LayerNorm(d_model)

    def forward(self, x):
        return self._forward(x, owned=False)

    def _forward(self, x, owned, then=None):
        """forward; with ``owned`` (x is a temporary of the caller's, e.g. the LM's embedding
        output) an inference forward whose rows need no padding updates x itself as the
        residual stream instead of a copy of it.  ``then`` (an nn.LayerNorm, the LM's norm_f)
        is applied after norm_final, in inference as one fused pass over the rows."""
        _ops._on_gpu(x)
        chunks = {layer.chunk_size for layer in self.layers}
        if torch.is_grad_enabled() or len(chunks) != 1 or self.training:
            for layer in self.layers:
                x, _ = layer(x)
        else:
            # Inference: one residual stream updated in place by every block.  Each block
            # of the reference left-pads its own input with zero rows (model.py:388-389), so
            # the pad rows are zeroed again before every block.
            (C,) = chunks
            B, L, dm = x.shape
            pad = (C - L % C) % C
            if owned and pad == 0 and x.is_contiguous():
                r = x
            else:
                r = torch.empty(B, L + pad, dm, device=x.device, dtype=x.dtype)
                r[:, pad:].copy_(x)
            for layer in self.layers:
                if pad:
                    r[:, :pad].zero_()
                layer._residual_step_(r)
            x = r[:, pad:]
            if then is not None and _ops.layer_norm2_ok(x):
                nf = self.norm_final
                return _ops.layer_norm2(x.contiguous(), nf.weight, nf.bias, nf.eps, then.weight, then.bias, then.eps)
        x = layer_norm(x, self.norm_final.weight, self.norm_final.bias, self.norm_final.eps)
        return x if then is None else layer_norm(x, then.weight, then.bias, then.eps)

    def prefill(self, x):
        """Forward over x [B,L,dm] (inference) that also returns every block's BlockState."""
        _ops._on_gpu(x)
        chunks = {layer.chunk_size for layer in self.layers}
        if len(chunks) != 1:
            raise RuntimeError("prefill needs one chunk size for all blocks")
        (C,) = chunks
        B, L, dm = x.shape
        pad = (C - L % C) % C
        r = torch.empty(B, L + pad, dm, device=x.device, dtype=x.dtype)
        r[:, pad:].copy_(x)
        states = []
        with torch.no_grad():
            for layer in self.layers:
                if pad:
                    r[:, :pad].zero_()
                st = layer.new_state(B, x.device, x.dtype)
                layer._residual_step_(r, st)
                states.append(st)
        y = _ops.layer_norm(r[:, pad:].contiguous(), self.norm_final.weight, self.norm_final.bias,
                            self.norm_final.eps)
        return y, states

    def step(self, x, states, pos_dev=None, then=None):
        """One token per batch row through every block and norm_final: x [B,dm] -> [B,dm].
        ``then`` (an nn.LayerNorm, the LM's norm_f) is applied after norm_final in the same
        pass (hdcm_rowln2_fwd, bit-identical to two LayerNorm launches)."""
        with torch.no_grad():
            for layer, st in zip(self.layers, states):
                x = layer.step(x, st, pos_dev)
        nf = self.norm_final
        if then is not None and _ops.layer_norm2_ok(x):
            return _ops.layer_norm2(x.contiguous(), nf.weight, nf.bias, nf.eps, then.weight, then.bias, then.eps)
        x = _ops.layer_norm(x, nf.weight, nf.bias, nf.eps)
        return x if then is None else _ops.layer_norm(x, then.weight, then.bias, then.eps)


def set_fused_out_proj(module, enabled=True):
    """Switch the folded LayerNorm + out_proj GEMM of every HdcMamba9v3Block inside
    ``module`` on or off; returns ``module``."""
    for m in module.modules():
        if isinstance(m, HdcMamba9v3Block):
            m.fused_out_proj = bool(enabled)
    return module


def set_fused_step_front(module, enabled=True):
    """Switch the one-launch LayerNorm + conv + in_proj of the decode step of every
    HdcMamba9v3Block inside ``module`` on or off; returns ``module``."""
    for m in module.modules():
        if isinstance(m, HdcMamba9v3Block):
            m.fused_step_front = bool(enabled)
    return module


def set_differentiable_mixer(module, enabled=True):
    """Switch every HdcMamba9v3Block inside ``module`` to (or back from) the differentiable
    mixer; returns ``module``."""
    for m in module.modules():
        if isinstance(m, HdcMamba9v3Block):
            m.differentiable_mixer = bool(enabled)
    return module
