"""Seeded inputs and weight recipes for the workloads the parity tests and bench use.

Workloads (all chunk 64 unless stated):
  block_c1  one block, fp32, B=1 L=256 d_model=256 d_state=64 heads=8
  block_c2  one block, bf16, B=4 L=2048 d_model=768 d_state=64 heads=8, SSM and slot
            decays drawn uniformly in [0.9, 0.999]
  lm_c3     12 layers d_model=768 d_state=64 heads=12 vocab 50304, B=8 L=4096
  lm_c4     24 layers d_model=1024 d_state=128 heads=16 vocab 50304, B=1 L=32768
"""
from __future__ import annotations

import torch

VOCAB = 50304

WORKLOADS = {
    "block_c1": dict(d_model=256, d_state=64, num_heads=8, chunk=64, B=1, L=256, dtype=torch.float32),
    "block_c2": dict(d_model=768, d_state=64, num_heads=8, chunk=64, B=4, L=2048, dtype=torch.bfloat16),
    "lm_c3": dict(d_model=768, d_state=64, num_heads=12, chunk=64, n_layers=12, B=8, L=4096,
                  dtype=torch.bfloat16),
    "lm_c4": dict(d_model=1024, d_state=128, num_heads=16, chunk=64, n_layers=24, B=1, L=32768,
                  dtype=torch.bfloat16),
    # prefill B=16 x 8192, then 256 single-token decode steps
    "lm_c5": dict(d_model=2048, d_state=128, num_heads=32, chunk=64, n_layers=48, B=16, L=8192,
                  decode_steps=256, dtype=torch.bfloat16),
}


def reinit_block_(blk, seed=0, decays_uniform=False):
    """Weights N(0, 0.02) for the linear/conv weights and biases, LN/GN at 1/0; A_log,
    decay_log and the dt bias keep the constructor values.  With ``decays_uniform`` the
    SSM per-channel decay exp(dt*A) and the slot gamma are drawn from U[0.9, 0.999]."""
    g = torch.Generator().manual_seed(seed)
    ds = blk.d_state
    with torch.no_grad():
        for t in (blk.conv1d.weight, blk.conv1d.bias, blk.out_proj.weight):
            t.copy_(torch.randn(t.shape, generator=g) * 0.02)
        w = torch.randn(blk.in_proj.weight.shape, generator=g) * 0.02
        blk.in_proj.weight.copy_(w)
        b = torch.randn(blk.in_proj.bias.shape, generator=g) * 0.02
        b[:ds] = blk.in_proj.bias[:ds]
        blk.in_proj.bias.copy_(b)
        blk.norm.weight.fill_(1.0); blk.norm.bias.zero_()
        blk.group_norm.weight.fill_(1.0); blk.group_norm.bias.zero_()
        if decays_uniform:
            u = 0.9 + 0.099 * torch.rand(ds, generator=g)
            dt = -torch.log(u) / torch.exp(blk.A_log.float())
            blk.in_proj.bias[:ds] = torch.log(torch.expm1(dt))
            blk.in_proj.weight[:ds] *= 0.1  # N(0, 0.002): dt stays token dependent
            gam = 0.9 + 0.099 * torch.rand(blk.num_heads, generator=g)
            blk.decay_log.copy_(torch.log(1.0 / gam - 1.0))
        blk.gamma_buf.copy_(torch.exp(-torch.nn.functional.softplus(blk.decay_log)))
    return blk


def make_block(name, seed=0):
    from hdcmamba_amd import HdcMamba9v3Block

    cfg = WORKLOADS[name]
    torch.manual_seed(seed)
    blk = HdcMamba9v3Block(cfg["d_model"], cfg["d_state"], cfg["num_heads"], cfg["chunk"])
    reinit_block_(blk, seed, decays_uniform=(name == "block_c2"))
    return blk.eval()


def block_input(name, seed=1):
    cfg = WORKLOADS[name]
    g = torch.Generator().manual_seed(seed)
    return torch.randn(cfg["B"], cfg["L"], cfg["d_model"], generator=g).to(cfg["dtype"])


def make_lm(name, seed=0, n_layers=None):
    from hdcmamba_amd import HdcMambaLM

    cfg = WORKLOADS[name]
    torch.manual_seed(seed)
    return HdcMambaLM(cfg["d_model"], n_layers or cfg["n_layers"], cfg["d_state"], cfg["num_heads"],
                      vocab_size=VOCAB, chunk_size=cfg["chunk"]).eval()


def lm_input(name, seed=1, B=None, L=None):
    cfg = WORKLOADS[name]
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, VOCAB, (B or cfg["B"], L or cfg["L"]), generator=g)


def oracle_cfg(blk):
    from oracle import BlockCfg

    return BlockCfg(blk.d_model, blk.d_state, blk.num_heads, blk.chunk_size)


def slot_inputs(B, L, dm, ds, H, dtype, seed=0, gamma_lo=0.9, gamma_hi=0.999):
    """Random projs rows plus per-head decays and GroupNorm affine for slot tests."""
    g = torch.Generator().manual_seed(seed)
    P = 3 * ds + 4 * dm
    projs = torch.randn(B, L, P, generator=g).to(dtype)
    gamma = (gamma_lo + (gamma_hi - gamma_lo) * torch.rand(H, generator=g)).to(dtype)
    gn_w = (1.0 + 0.1 * torch.randn(dm, generator=g)).to(dtype)
    gn_b = (0.1 * torch.randn(dm, generator=g)).to(dtype)
    return projs, gamma, gn_w, gn_b


def ssm_inputs(B, L, ds, dtype, extra_cols=8, seed=0):
    """projs rows whose dt columns give dt in roughly [0.001, 0.1], plus a few large dt_raw
    values (> 20) to cover the softplus threshold."""
    g = torch.Generator().manual_seed(seed)
    P = 3 * ds + extra_cols
    projs = torch.randn(B, L, P, generator=g)
    dt0 = 0.001 + 0.099 * torch.rand(B, L, ds, generator=g)
    projs[..., :ds] = torch.log(torch.expm1(dt0)) + 0.3 * torch.randn(B, L, ds, generator=g)
    projs[0, min(3, L - 1), :4] = 25.0
    A_log = torch.log(torch.linspace(0.99, 0.9999, ds))
    return projs.to(dtype), A_log.to(dtype)


def tol(dtype):
    return (1e-4, 1e-4) if dtype == torch.float32 else (2e-2, 2e-2)


def max_rel(got, ref):
    got, ref = got.float().cpu(), ref.float().cpu()
    return ((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def assert_close(got, ref, dtype, what=""):
    """Elementwise |got-ref| <= atol + rtol*|ref| (fp32 1e-4/1e-4, bf16 2e-2/2e-2) and, for bf16,
    also the relative bound max|got-ref| <= 2e-2 max|ref|: together no looser than either
    the elementwise or the normwise reading of "2e-2 relative"."""
    atol, rtol = tol(dtype)
    torch.testing.assert_close(got.float().cpu(), ref.float().cpu(), atol=atol, rtol=rtol,
                               msg=lambda m: f"{what}: {m}")
    if dtype != torch.float32 and got.numel() > 0:
        r = max_rel(got, ref)
        assert r <= 2e-2, f"{what}: normwise max-abs/max|ref| = {r:.3e} > 2e-2"


def assert_close_normwise(got, ref, dtype, what=""):
    """Max-abs error relative to the reference's max magnitude: <= 1e-4 (fp32), 2e-2 (bf16).
    Used for end-to-end outputs, where bf16 rounding flips compound through several
    layers and an elementwise bound is dominated by near-zero entries."""
    lim = 1e-4 if dtype == torch.float32 else 2e-2
    r = max_rel(got, ref)
    assert r <= lim, f"{what}: normwise max-abs/max|ref| = {r:.3e} > {lim}"

