"""CPU oracle for the HdcMamba block forward -- TEST INFRASTRUCTURE ONLY.

This module restates, in plain PyTorch on the CPU, what the reference computes on
its forward path (N01N9/hdcmamba, ``hdcmamba/model.py``).  It is the checker the
HIP kernels are compared against; only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg may import it.  The product package
(``hdcmamba_amd``) never imports it and has no CPU fallback.

Two semantics are provided:

* ``"intended"`` (default): what the reference module means to compute.  Every
  internal quantity stays fp32 and is rounded to the activation dtype only where a
  tensor is materialised (projs, the concatenated ``combined`` row, the block
  output).  Operands of the reference's ``tl.dot`` calls are rounded to the
  activation dtype exactly where the reference rounds them (model.py:263,265,268,
  271), which is a no-op in fp32.
* ``"faithful"``: additionally reproduces the reference kernels' deterministic
  defects -- the gate/y_ssm launch strides (model.py:377), the 128-position chunk
  map in the gate kernel (model.py:288), the constant-one padding features when
  ``head_dim`` is not a power of two >= 64 (model.py:245-262,290) and the bf16
  rounding of SSM intermediates and of the gated slot output even for fp32
  inputs (model.py:196-198,209,233,293).  Chunk sizes above 128 read memory the
  reference never wrote (model.py:17,245-246) and are rejected.

Parity status of each function (how it is pinned, see tests/test_oracle_*.py):

* ``norm_conv``      -- pinned: F.layer_norm + F.conv1d library routines, identity-tap KAT.
* ``ssm_sequential`` -- pinned: closed form for constant inputs, brute-force Python loop.
* ``ssm_chunked``    -- pinned: equals ``ssm_sequential`` for several chunk sizes.
* ``slot_sequential``-- pinned: hand-computed two-token KAT of the cross-chunk rule,
  C=L reduces to masked decayed attention, gamma=1 reduces to a cumulative sum.
* ``slot_chunked``   -- pinned: equals ``slot_sequential`` (fp32) for several chunk sizes;
  its bf16 rounding points (phi(q), phi(k), the decayed masked scores, phi(q)*gamma^c,
  phi(k)*gamma^(C-1-c), the carried state) against the reference's own bf16 block forward
  (its kernels under Triton's CPU interpreter with bf16 dot operands widened to fp32): the
  oracle matches those vectors, and leaving any one rounding point out does not.
* ``gnorm_gate``     -- pinned: F.group_norm per token + torch.sigmoid.
* ``rowln``          -- pinned: F.layer_norm.
* ``block_forward_stream`` -- pinned: equals ``block_forward`` when the whole sequence is
  the prefill, and row by row equals a sequential recurrence over the padded sequence
  (every stage is causal, so right padding changes no kept row).
* ``block_prefill_state`` / ``block_step`` -- pinned: a prefill followed by steps equals
  ``block_forward_stream`` over the same rows (fp32 1e-4, chunk ends and left-padded
  prefills included); a planted slip in the chunk-end fold fails it.
* faithful-mode address maps (B1-B3, B5) -- pinned by hand-computed index KATs
  restated from the launch arguments and by the reference's own kernels run under
  Triton's CPU interpreter on the five fp32 block vectors (batch 2, chunk 128, head
  dim 96, ragged length 100): the faithful oracle matches them within 5e-4 normwise,
  the intended semantics miss every one by more than 1e-2.  The reference is never run
  on a GPU (it needs CUDA).
* ``model_forward`` -- pinned: the reference's own model forward (two fp32 blocks at chunk
  64, head dim 32, under Triton's CPU interpreter) matches the faithful oracle within 2e-8;
  the blocks in the other order, or without norm_final, miss it.
* ``lm_forward`` -- by construction: embedding, ``model_forward``, norm_f and the tied head
  (F.embedding, F.layer_norm, F.linear); the reference's LM wrapper cannot be imported here
  (train_fineweb.py needs wandb).
* constructor RNG order -- pinned by the fixture in tests/golden (see its script).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

__all__ = [
    "BlockCfg", "kernel_rounding", "skip_slot_rounding", "SLOT_ROUNDING_SITES", "softplus20", "phi", "norm_conv", "ssm_sequential", "ssm_chunked",
    "slot_sequential", "slot_chunked", "attend_sequential", "attend_chunked", "gnorm_gate", "rowln", "block_forward", "block_forward_stream",
    "block_prefill_state", "block_step", "model_forward", "lm_forward", "init_block_params",
]


@dataclass(frozen=True)
class BlockCfg:
    d_model: int
    d_state: int
    num_heads: int
    chunk_size: int

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads

    @property
    def proj_width(self) -> int:
        return 3 * self.d_state + 4 * self.d_model


# Rounding applied where the reference's Triton kernels convert fp32 values to bf16
# (operand casts and stores).  "rne" is what a GPU does; "trunc" is what Triton's CPU
# interpreter does (it drops the low 16 bits), used only to compare against vectors the
# reference produced under the interpreter.  Rounding done by torch ops (F.linear,
# F.layer_norm(...).to, the residual add) is always round-to-nearest-even.
_KERNEL_ROUNDING = "rne"


class kernel_rounding:
    """Context manager selecting the kernel-side bf16 rounding mode ("rne" or "trunc")."""

    def __init__(self, mode: str):
        assert mode in ("rne", "trunc")
        self.mode = mode

    def __enter__(self):
        global _KERNEL_ROUNDING
        self.prev, _KERNEL_ROUNDING = _KERNEL_ROUNDING, self.mode
        return self

    def __exit__(self, *exc):
        global _KERNEL_ROUNDING
        _KERNEL_ROUNDING = self.prev


# The slot recurrence's rounding points, named for the checks that leave one out to show
# that the reference's bf16 vectors tell it apart (tests/test_oracle_reference.py).
SLOT_ROUNDING_SITES = ("phi_q", "phi_k", "scores", "q_decay", "k_decay", "state")
_SKIPPED_SITES: frozenset = frozenset()


class skip_slot_rounding:
    """Context manager that leaves the named slot rounding points out (checks only)."""

    def __init__(self, *sites: str):
        assert all(x in SLOT_ROUNDING_SITES for x in sites), sites
        self.sites = frozenset(sites)

    def __enter__(self):
        global _SKIPPED_SITES
        self.prev, _SKIPPED_SITES = _SKIPPED_SITES, self.sites
        return self

    def __exit__(self, *exc):
        global _SKIPPED_SITES
        _SKIPPED_SITES = self.prev


def _rnd(t: torch.Tensor, dtype: torch.dtype, site: str | None = None) -> torch.Tensor:
    """Kernel-side rounding of fp32 values to ``dtype``, returned as fp32 (no-op for fp32).
    ``site`` names a slot rounding point that skip_slot_rounding can leave out."""
    if dtype == torch.float32 or (site is not None and site in _SKIPPED_SITES):
        return t.float()
    if _KERNEL_ROUNDING == "trunc" and dtype == torch.bfloat16:
        return (t.float().contiguous().view(torch.int32) & ~0xFFFF).view(torch.float32)
    return t.to(dtype).float()


def softplus20(x: torch.Tensor) -> torch.Tensor:
    """softplus with threshold 20 as written at model.py:192 and 229: log(1+exp(x))."""
    return torch.where(x > 20.0, x, torch.log(1.0 + torch.exp(x)))


def phi(z: torch.Tensor) -> torch.Tensor:
    """Feature map elu(z)+1 as written at model.py:261-262."""
    return torch.where(z > 0, z + 1.0, torch.exp(z))


# --------------------------------------------------------------------------------------
# LayerNorm + causal depthwise conv (model.py:22-72, 126-146, 168-172)
# --------------------------------------------------------------------------------------
def norm_conv(x, ln_w, ln_b, conv_w, conv_b, eps):
    """out[t] = sum_k u[t-3+k] * w[:,k] + b, u = LayerNorm(x) with biased variance.

    Rows t<0 are LayerNorm of a zero row, i.e. the LN bias (model.py:47-54).
    ``conv_w`` is [D,4] (``conv1d.weight.squeeze(1)``).  Math in fp32, output in x.dtype
    (model.py:62-71).
    """
    dtype = x.dtype
    xf = x.float()
    B, L, D = xf.shape
    w = ln_w.to(dtype).float()
    b = ln_b.to(dtype).float()
    cw = conv_w.to(dtype).float()
    cb = conv_b.to(dtype).float()
    mean = xf.mean(-1, keepdim=True)
    xc = xf - mean
    var = (xc * xc).mean(-1, keepdim=True)
    u = xc * torch.rsqrt(var + eps) * w + b
    up = torch.cat([b.expand(B, 3, D), u], dim=1)
    out = (up[:, 0:L] * cw[:, 0] + up[:, 1:L + 1] * cw[:, 1]
           + up[:, 2:L + 2] * cw[:, 2] + up[:, 3:L + 3] * cw[:, 3] + cb)
    return _rnd(out, dtype).to(dtype)


# --------------------------------------------------------------------------------------
# Selective scan over d_state channels (model.py:175-233)
# --------------------------------------------------------------------------------------
def _ssm_inputs(projs, A_log, ds):
    dt_raw = projs[..., 0:ds].float()
    xs = projs[..., ds:2 * ds].float()
    bs = projs[..., 2 * ds:3 * ds].float()
    A = -torch.exp(A_log.float())
    dt = softplus20(dt_raw)
    return dt, dt * A, dt * bs * xs  # dt, log-decay, input term (model.py:192-195)


def ssm_sequential(projs, A_log, ds, h0=None):
    """Direct per-token recurrence h_t = h_{t-1} * exp(ld_t) + dt_t*b_t*x_t, y_t = h_t.

    Returns (y fp32 [B,L,ds], h_final fp32 [B,ds]).
    """
    _, ld, u = _ssm_inputs(projs, A_log, ds)
    B, L, _ = ld.shape
    h = torch.zeros(B, ds) if h0 is None else h0.float().clone()
    y = torch.empty(B, L, ds)
    for t in range(L):
        h = h * torch.exp(ld[:, t]) + u[:, t]
        y[:, t] = h
    return y, h


def ssm_chunked(projs, A_log, ds, C, dtype=torch.float32, semantics="intended", h0=None):
    """Chunked form of the scan as the reference launches it (model.py:345-363).

    intra (model.py:187-198): per chunk, h from 0; y_intra, last state, sum of log decays.
    scan  (model.py:207-212): G[n] = carried state before chunk n.
    inter (model.py:226-233): y = y_intra + G[n] * exp(cumsum(ld)).
    Faithful mode rounds y_intra/last/sum(ld)/G and y to bf16 as the kernels store them.
    Returns (y fp32 [B,L,ds], h_final fp32 [B,ds]).
    """
    _, ld, u = _ssm_inputs(projs, A_log, ds)
    B, L, _ = ld.shape
    assert L % C == 0
    N = L // C
    ld = ld.view(B, N, C, ds)
    u = u.view(B, N, C, ds)
    bf = (lambda t: _rnd(t, torch.bfloat16)) if semantics == "faithful" else (lambda t: t)
    acc = torch.zeros(B, N, ds)
    sld = torch.zeros(B, N, ds)
    y_intra = torch.empty(B, N, C, ds)
    for c in range(C):
        sld = sld + ld[:, :, c]
        acc = acc * torch.exp(ld[:, :, c]) + u[:, :, c]
        y_intra[:, :, c] = acc
    y_intra, last, sld = bf(y_intra), bf(acc), bf(sld)
    state = torch.zeros(B, ds) if h0 is None else h0.float().clone()
    G = torch.empty(B, N, ds)
    for n in range(N):
        G[:, n] = bf(state)
        state = state * torch.exp(sld[:, n]) + last[:, n]
    cum = torch.zeros(B, N, ds)
    y = torch.empty(B, N, C, ds)
    for c in range(C):
        cum = cum + ld[:, :, c]
        y[:, :, c] = bf(y_intra[:, :, c] + G * torch.exp(cum))
    return y.view(B, L, ds), state


# --------------------------------------------------------------------------------------
# Slot memory: per-head decayed linear attention (model.py:236-272)
# --------------------------------------------------------------------------------------
def _slot_qkv(projs, dm, ds, H):
    B, L, _ = projs.shape
    hd = dm // H
    off = 3 * ds
    q = projs[..., off:off + dm].float().view(B, L, H, hd)
    k = projs[..., off + dm:off + 2 * dm].float().view(B, L, H, hd)
    v = projs[..., off + 2 * dm:off + 3 * dm].float().view(B, L, H, hd)
    return q, k, v


def slot_sequential(projs, gamma, dm, ds, H, C):
    """Brute-force y_t = sum_{j<=t} w(t,j) (phi(q_t).phi(k_j)) v_j, fp32, small inputs only.

    w(t,j) = gamma^(t-j) when j is in t's chunk and gamma^(t-j-1) otherwise
    (model.py:265 for the intra-chunk part, model.py:267-268 + 271-272 for the carry).
    Returns y fp32 [B,L,H,hd].
    """
    q, k, v = _slot_qkv(projs, dm, ds, H)
    q, k = phi(q), phi(k)
    B, L, _, hd = q.shape
    g = gamma.float()
    y = torch.zeros(B, L, H, hd)
    for t in range(L):
        for j in range(t + 1):
            e = (t - j) - (0 if t // C == j // C else 1)
            w = g ** e  # [H]
            s = (q[:, t] * k[:, j]).sum(-1) * w  # [B,H]
            y[:, t] += s[..., None] * v[:, j]
    return y


def slot_chunked(projs, gamma, dm, ds, H, C, dtype=torch.float32, semantics="intended", S0=None):
    """Chunked slot recurrence exactly as model.py:254-272 orders it.

    Operands of each dot are rounded to ``dtype`` where the reference rounds them.
    In faithful mode, heads with head_dim below max(64, next_pow2(head_dim)) get the
    reference's constant-one padding features (masked loads of 0 map to phi(0)=1).
    Returns (y fp32 [B,L,H,hd], running state fp32 [B,H,hdk,hd]).
    """
    q, k, v = _slot_qkv(projs, dm, ds, H)
    B, L, _, hd = q.shape
    assert L % C == 0
    qf = _rnd(phi(q), dtype, "phi_q")
    kf = _rnd(phi(k), dtype, "phi_k")
    if semantics == "faithful":
        blk = max(64, 1 << (hd - 1).bit_length())
        if blk > hd:
            ones = torch.ones(B, L, H, blk - hd)
            qf = torch.cat([qf, ones], -1)
            kf = torch.cat([kf, ones], -1)
    return attend_chunked(qf, kf, v, gamma, C, dtype, S0)


def attend_sequential(qf, kf, v, gamma, C):
    """Brute-force y_t = sum_{j<=t} w(t,j) (qf_t.kf_j) v_j on featured q/k [B,L,H,hk] and
    v [B,L,H,hd], with the slot weights w(t,j) = gamma^(t-j) in t's chunk and
    gamma^(t-j-1) across chunks (model.py:265-272).  fp32, small inputs only."""
    B, L, H, _ = qf.shape
    g = gamma.float()
    y = torch.zeros(B, L, H, v.shape[-1])
    for t in range(L):
        for j in range(t + 1):
            e = (t - j) - (0 if t // C == j // C else 1)
            s = (qf[:, t].float() * kf[:, j].float()).sum(-1) * g ** e  # [B,H]
            y[:, t] += s[..., None] * v[:, j].float()
    return y


def attend_chunked(qf, kf, v, gamma, C, dtype=torch.float32, S0=None):
    """The slot recurrence of slot_chunked on already featured q/k [B,L,H,hk] (phi(q),
    phi(k), or any other tensors) and v [B,L,H,hd], chunked as model.py:254-272 orders it;
    dot operands rounded to ``dtype`` where the reference rounds them.
    Returns (y fp32 [B,L,H,hd], running state fp32 [B,H,hk,hd])."""
    B, L, H, hk = qf.shape
    hd = v.shape[-1]
    assert L % C == 0
    N = L // C
    # [B,H,N,C,*]
    qf = _rnd(qf.float(), dtype, "phi_q").view(B, N, C, H, hk).permute(0, 3, 1, 2, 4)
    kf = _rnd(kf.float(), dtype, "phi_k").view(B, N, C, H, hk).permute(0, 3, 1, 2, 4)
    vv = v.float().view(B, N, C, H, hd).permute(0, 3, 1, 2, 4)
    lg = torch.log(gamma.float()).view(1, H, 1, 1, 1)
    idx = torch.arange(C, dtype=torch.float32)
    diff = idx[:, None] - idx[None, :]
    causal = diff >= 0
    decay = torch.exp(diff * lg)  # [1,H,1,C,C]
    scores = qf @ kf.transpose(-1, -2)
    scores = _rnd(torch.where(causal, scores * decay, torch.zeros(())), dtype, "scores")
    y_intra = scores @ vv
    q_decay = torch.exp(idx.view(1, 1, 1, C, 1) * lg)
    k_decay = torch.exp((C - 1 - idx).view(1, 1, 1, C, 1) * lg)
    qd = _rnd(qf * q_decay, dtype, "q_decay")
    kd = _rnd(kf * k_decay, dtype, "k_decay")
    U = kd.transpose(-1, -2) @ vv  # [B,H,N,hk,hd]
    gC = torch.exp(C * lg.view(1, H, 1, 1))
    running = torch.zeros(B, H, hk, hd) if S0 is None else S0.float().clone()
    y_inter = torch.empty_like(y_intra)
    for n in range(N):
        y_inter[:, :, n] = qd[:, :, n] @ _rnd(running, dtype, "state")
        running = running * gC + U[:, :, n]
    y = (y_intra + y_inter).permute(0, 2, 3, 1, 4).reshape(B, L, H, hd)
    return y, running


# --------------------------------------------------------------------------------------
# Per-token-per-head GroupNorm + sigmoid gate (model.py:274-295), row LayerNorm (model.py:382)
# --------------------------------------------------------------------------------------
def gnorm_gate(y, gate, gn_w, gn_b, H, eps=1e-5, pad_block=None):
    """out = ((y-mu)/sqrt(var+eps) * w + b) * sigmoid(gate), statistics per (token, head).

    ``y`` fp32 [B,L,H,hd]; ``gate`` [B,L,H*hd]; returns fp32 [B,L,H*hd].
    ``pad_block`` (faithful mode) adds the (pad_block-hd)*mu^2/hd variance term of
    the reference's unmasked centred lanes (model.py:290).
    """
    B, L, _, hd = y.shape
    mean = y.mean(-1, keepdim=True)
    yc = y - mean
    var = (yc * yc).mean(-1, keepdim=True)
    if pad_block is not None and pad_block > hd:
        var = var + (pad_block - hd) * mean * mean / hd
    w = gn_w.float().view(H, hd)
    b = gn_b.float().view(H, hd)
    ygn = yc / torch.sqrt(var + eps) * w + b
    g = gate.float().view(B, L, H, hd)
    out = ygn * (1.0 / (1.0 + torch.exp(-g)))
    return out.reshape(B, L, H * hd)


def rowln(x, w=None, b=None, eps=1e-5):
    """LayerNorm over the last dim in fp32, output in x.dtype (model.py:382, nn.LayerNorm)."""
    xf = x.float()
    mean = xf.mean(-1, keepdim=True)
    xc = xf - mean
    var = (xc * xc).mean(-1, keepdim=True)
    out = xc * torch.rsqrt(var + eps)
    if w is not None:
        out = out * w.float()
    if b is not None:
        out = out + b.float()
    return out.to(x.dtype)


# --------------------------------------------------------------------------------------
# Faithful-mode address maps of the gate kernel launch (model.py:373-380, 288)
# --------------------------------------------------------------------------------------
def faithful_gate_index(B, L, dm, ds):
    """Flat projs index the reference reads for gate[b,l,j]: its launch passes
    stride_b=B*L and stride_l=4*dm for a view whose true strides are L*P and P
    (model.py:373,377)."""
    b = torch.arange(B).view(B, 1, 1)
    l = torch.arange(L).view(1, L, 1)
    j = torch.arange(dm).view(1, 1, dm)
    return (3 * ds + 3 * dm) + b * (B * L) + l * (4 * dm) + j


def faithful_yssm_index(B, L, ds):
    """Flat y_ssm index read for token (b,l) channel d: batch stride passed as B*L
    instead of L*ds (model.py:377)."""
    b = torch.arange(B).view(B, 1, 1)
    l = torch.arange(L).view(1, L, 1)
    d = torch.arange(ds).view(1, 1, ds)
    return b * (B * L) + l * ds + d


def faithful_slot_position(L, C):
    """Position within a head's flattened [N,C] y_slot read for token l: the gate kernel
    computes (l//128, l%128) as (chunk, offset) whatever C is (model.py:288)."""
    l = torch.arange(L)
    return (l // 128) * C + (l % 128)


# --------------------------------------------------------------------------------------
# Block / model / LM forward (model.py:331-404, train_fineweb.py:86-94)
# --------------------------------------------------------------------------------------
def block_forward(p, x, cfg: BlockCfg, semantics="intended", eps=1e-5, return_states=False, mixer_grad=False):
    """One HdcMamba9v3Block forward in eval mode (model.py:386-394 + 331-384).

    ``p`` is the block's state_dict (tensors in the model dtype); ``x`` is [B,L,D].
    L is left-padded with zero rows to a multiple of the chunk (model.py:388-389).
    The reference's SSM, slot and gate kernels have no autograd (model.py:340-384), so
    its ``combined`` buffer is a constant for backward: only out_proj, the residual
    stream and what follows the blocks receive gradients.  Autograd through this function
    reproduces that (``combined`` is detached) unless ``mixer_grad`` is set.
    """
    C = cfg.chunk_size
    pad = (C - x.shape[1] % C) % C
    return _block_padded(p, x, cfg, pad, 0, semantics, eps, return_states, mixer_grad)


def block_forward_stream(p, x, cfg: BlockCfg, n_prefill, eps=1e-5):
    """A prefill of x[:, :n_prefill] continued token by token over the remaining rows
    (intended semantics): the chunk grid is the prefill's (left pad to a multiple of C),
    and the sequence is right-padded to a whole chunk.  Every stage is causal, so the
    right padding changes no kept row.  Returns [B,L,D]."""
    C = cfg.chunk_size
    pad_l = (C - n_prefill % C) % C
    pad_r = (C - (pad_l + x.shape[1]) % C) % C
    return _block_padded(p, x, cfg, pad_l, pad_r, "intended", eps, False)


def _block_padded(p, x, cfg, pad, pad_r, semantics, eps, return_states, mixer_grad=False):
    dtype = x.dtype
    dm, ds, H, C = cfg.d_model, cfg.d_state, cfg.num_heads, cfg.chunk_size
    hd = cfg.head_dim
    if semantics == "faithful" and C > 128:
        raise ValueError("faithful semantics undefined for chunk_size > 128 (model.py:17,245-246)")
    B, L_in, _ = x.shape
    if pad or pad_r:
        x = F.pad(x, (0, 0, pad, pad_r))
    L = x.shape[1]
    x_conv = norm_conv(x, p["norm.weight"], p["norm.bias"], p["conv1d.weight"].squeeze(1),
                       p["conv1d.bias"], eps)
    projs = F.linear(x_conv, p["in_proj.weight"].to(dtype), p["in_proj.bias"].to(dtype))
    y_ssm, h_fin = ssm_chunked(projs, p["A_log"].to(dtype), ds, C, dtype, semantics)
    gamma = p["gamma_buf"].to(dtype)
    y_slot, s_fin = slot_chunked(projs, gamma, dm, ds, H, C, dtype, semantics)
    gate = projs[..., 3 * ds + 3 * dm:]
    if semantics == "faithful":
        flat = projs.reshape(-1)
        gate = flat[faithful_gate_index(B, L, dm, ds)]
        pos = faithful_slot_position(L, C)
        y_slot = _rnd(y_slot, dtype)[:, pos]
        y_ssm_t = _rnd(y_ssm, dtype).reshape(-1)[faithful_yssm_index(B, L, ds)]
        blk = max(64, 1 << (hd - 1).bit_length())
        g = _rnd(gnorm_gate(y_slot, gate, p["group_norm.weight"], p["group_norm.bias"], H,
                            pad_block=blk), torch.bfloat16)
    else:
        y_ssm_t = y_ssm
        g = gnorm_gate(y_slot, gate, p["group_norm.weight"], p["group_norm.bias"], H)
    combined = torch.cat([_rnd(y_ssm_t, dtype), _rnd(g, dtype)], -1).to(dtype)
    if not mixer_grad:
        combined = combined.detach()
    c = F.layer_norm(combined.float(), (ds + dm,)).to(dtype)
    res = F.linear(c, p["out_proj.weight"].to(dtype))
    out = (x + res)[:, pad:pad + L_in, :]
    if return_states:
        return out, {"h": h_fin, "S": s_fin, "projs": projs, "combined": combined, "x_conv": x_conv}
    return out


def block_prefill_state(p, x, cfg: BlockCfg, eps=1e-5):
    """block_forward over a prefill x [B,L,D] and the state it leaves for block_step:
    ``conv`` the last three block-input rows (zero rows before the sequence start, whose
    LayerNorm is the LN bias as in norm_conv), ``h`` the SSM state, ``S_prev`` the slot state
    at the chunk boundary the left-padded prefill ends on, ``S_intra`` (unused at offset 0)
    and the chunk offset ``pos`` = 0.  Returns (out [B,L,D], state)."""
    out, st = block_forward(p, x, cfg, eps=eps, return_states=True)
    B, _, D = x.shape
    H, hd = cfg.num_heads, cfg.head_dim
    conv = torch.cat([torch.zeros(B, 3, D, dtype=x.dtype), x], 1)[:, -3:].clone()
    return out, {"conv": conv, "h": st["h"].float().clone(), "S_prev": st["S"].float().clone(),
                 "S_intra": torch.zeros(B, H, hd, hd), "pos": 0}


def block_step(p, x, state, cfg: BlockCfg, eps=1e-5):
    """One token per batch row after block_prefill_state: x [B,D] -> [B,D], ``state``
    advanced in place.  The chunked forward continued token by token (what
    block_forward_stream computes for the whole sequence; the reference has no recurrent
    step): the conv over the three history rows and the token, the SSM recurrence of
    ssm_sequential, and for the slot memory, with c the token's offset in its chunk,
      S_eff = S_prev + phi(k)^T v (c = 0),  gamma S_eff_prev + phi(k)^T v (c > 0),
      y = phi(q) S_eff,
    S_eff kept in S_intra between the tokens of a chunk and folded at the chunk's last token
    into S_prev <- S_eff + (gamma^C - gamma^(C-1)) S_prev = gamma^C S_prev + the chunk's own
    decayed sum (attend_chunked's running state).  phi(q) and phi(k) are rounded to the
    activation dtype as in the chunked form; the states stay fp32."""
    dtype = x.dtype
    dm, ds, H, C = cfg.d_model, cfg.d_state, cfg.num_heads, cfg.chunk_size
    hd = cfg.head_dim
    B = x.shape[0]
    rows = torch.cat([state["conv"], x[:, None]], 1)  # [B,4,D], oldest first
    xc = norm_conv(rows, p["norm.weight"], p["norm.bias"], p["conv1d.weight"].squeeze(1),
                   p["conv1d.bias"], eps)[:, 3]
    state["conv"] = rows[:, 1:].clone()
    projs = F.linear(xc, p["in_proj.weight"].to(dtype), p["in_proj.bias"].to(dtype))
    _, ld, u = _ssm_inputs(projs, p["A_log"].to(dtype), ds)
    h = state["h"] * torch.exp(ld) + u
    state["h"] = h
    off = 3 * ds
    qf = _rnd(phi(projs[:, off:off + dm].float()), dtype).view(B, H, hd)
    kf = _rnd(phi(projs[:, off + dm:off + 2 * dm].float()), dtype).view(B, H, hd)
    v = projs[:, off + 2 * dm:off + 3 * dm].float().view(B, H, hd)
    g = p["gamma_buf"].to(dtype).float().view(1, H, 1, 1)
    c = state["pos"]
    kv = kf[..., :, None] * v[..., None, :]
    S_eff = state["S_prev"] + kv if c == 0 else g * state["S_intra"] + kv
    y = (qf[..., :, None] * S_eff).sum(-2)  # [B,H,hd]
    if c == C - 1:
        state["S_prev"] = S_eff + (g ** C - g ** (C - 1)) * state["S_prev"]
    else:
        state["S_intra"] = S_eff
    state["pos"] = (c + 1) % C
    gate = projs[:, off + 3 * dm:]
    gg = gnorm_gate(y.view(B, 1, H, hd), gate.view(B, 1, dm), p["group_norm.weight"], p["group_norm.bias"], H)
    combined = torch.cat([_rnd(h, dtype), _rnd(gg[:, 0], dtype)], -1).to(dtype)
    cn = F.layer_norm(combined.float(), (ds + dm,)).to(dtype)
    return x + F.linear(cn, p["out_proj.weight"].to(dtype))


def _sub(sd, prefix):
    n = len(prefix)
    return {k[n:]: v for k, v in sd.items() if k.startswith(prefix)}


def model_forward(sd, x, cfg: BlockCfg, n_layers, semantics="intended", layers=None, n_prefill=None):
    """HdcMamba9v3Model.forward (model.py:402-404): blocks then norm_final.  With
    ``n_prefill``, the blocks run as a prefill of that many rows continued token by token
    (block_forward_stream)."""
    for i in (range(n_layers) if layers is None else layers):
        p = _sub(sd, f"layers.{i}.")
        x = block_forward(p, x, cfg, semantics) if n_prefill is None else block_forward_stream(p, x, cfg, n_prefill)
    return F.layer_norm(x, (cfg.d_model,), sd["norm_final.weight"], sd["norm_final.bias"], 1e-5)


def lm_forward(sd, ids, cfg: BlockCfg, n_layers, semantics="intended", layers=None, n_prefill=None,
               positions=None, return_hidden=False):
    """UniversalLM.forward, HdcMamba arm (train_fineweb.py:86-94): embedding, backbone,
    norm_f, tied lm_head.  ``n_prefill`` as in model_forward.  With ``positions`` (a list of
    token positions) the head runs on those positions only: logits [B, len(positions), V]
    (the backbone still runs over the whole sequence).  With ``return_hidden`` the result is
    (logits, h), h [B, L, d_model] the head's input (norm_f's output) at every position."""
    x = F.embedding(ids, sd["embedding.weight"])
    x = model_forward(_sub(sd, "backbone."), x, cfg, n_layers, semantics, layers, n_prefill)
    if return_hidden:
        h = F.layer_norm(x, (cfg.d_model,), sd["norm_f.weight"], sd["norm_f.bias"], 1e-5)
        hp = h if positions is None else h[:, list(positions)]
        return F.linear(hp, sd["embedding.weight"]), h
    if positions is not None:
        x = x[:, list(positions)]
    x = F.layer_norm(x, (cfg.d_model,), sd["norm_f.weight"], sd["norm_f.bias"], 1e-5)
    return F.linear(x, sd["embedding.weight"])


# --------------------------------------------------------------------------------------
# Seeded parameter construction in the reference's RNG order (model.py:300-327,
# train_fineweb.py:47-84).  Used by tests to build inputs independently of the product.
# --------------------------------------------------------------------------------------
def init_block_params(cfg: BlockCfg, generator_seed=None):
    """State dict of a freshly constructed block, consuming the global RNG in the order
    nn.Conv1d default init, normal_(std=.02), nn.Linear default init, torch.rand(ds),
    xavier_uniform_ on q/k/v rows, nn.Linear default init of out_proj (model.py:306-327)."""
    if generator_seed is not None:
        torch.manual_seed(generator_seed)
    dm, ds, H = cfg.d_model, cfg.d_state, cfg.num_heads
    P = cfg.proj_width
    conv = torch.nn.Conv1d(dm, dm, 4, groups=dm, padding=3, bias=True)
    with torch.no_grad():
        torch.nn.init.normal_(conv.weight, std=0.02)
        conv.weight[:, 0, -1] += 1.0
        conv.bias.fill_(0.0)
    lin = torch.nn.Linear(dm, P, bias=True)
    with torch.no_grad():
        dt0 = torch.rand(ds) * (0.1 - 0.001) + 0.001
        lin.bias[:ds] = torch.log(torch.exp(dt0) - 1.0)
        torch.nn.init.xavier_uniform_(lin.weight[3 * ds:3 * ds + 3 * dm])
        lin.bias[3 * ds + 3 * dm:].fill_(1.0)
    A_log = torch.log(torch.linspace(0.99, 0.9999, ds))
    decay_log = torch.log(torch.ones(H) * 0.05)
    out = torch.nn.Linear(ds + dm, dm, bias=False)
    return {
        "norm.weight": torch.ones(dm), "norm.bias": torch.zeros(dm),
        "conv1d.weight": conv.weight.detach().clone(), "conv1d.bias": conv.bias.detach().clone(),
        "in_proj.weight": lin.weight.detach().clone(), "in_proj.bias": lin.bias.detach().clone(),
        "A_log": A_log, "decay_log": decay_log,
        "out_proj.weight": out.weight.detach().clone(),
        "group_norm.weight": torch.ones(dm), "group_norm.bias": torch.zeros(dm),
        "gamma_buf": torch.exp(-F.softplus(decay_log)),
    }
