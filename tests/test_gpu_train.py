"""Training through the HIP path: the row LayerNorm backward against torch's fp32 autograd,
and one LM backward against autograd through the CPU oracle.

The reference's SSM, slot and gate kernels have no autograd, so its training updates
out_proj, the residual stream, norm_final, norm_f and the tied embedding only; the oracle's
``combined`` is detached the same way.  Tolerances (max-abs error over the reference's
max magnitude): fp32 1e-4, bf16 2e-2.
"""
import pytest
import torch
import torch.nn.functional as F

import oracle
from cfgs import max_rel, reinit_block_

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,W,affine", [(300, 1024, True), (5, 1152, False), (64, 2048, True),
                                           (1, 256, True), (0, 512, True), (2500, 768, True)])
def test_layer_norm_backward(dev, dtype, rows, W, affine):
    from hdcmamba_amd.model import layer_norm

    _say("layer_norm bwd", dtype, rows, W, affine)
    g = torch.Generator().manual_seed(rows + W)
    x = (2 * torch.randn(rows, W, generator=g) + 0.3).to(dtype)
    dy = torch.randn(rows, W, generator=g).to(dtype)
    w = (1 + 0.2 * torch.randn(W, generator=g)).to(dtype) if affine else None
    b = (0.1 * torch.randn(W, generator=g)).to(dtype) if affine else None
    # reference: torch fp32 autograd on the same (rounded) values
    xr = x.float().clone().requires_grad_(True)
    wr = w.float().clone().requires_grad_(True) if affine else None
    br = b.float().clone().requires_grad_(True) if affine else None
    F.layer_norm(xr, (W,), wr, br, 1e-5).backward(dy.float())
    xd = x.to(dev).detach().requires_grad_(True)
    wd = w.to(dev).detach().requires_grad_(True) if affine else None
    bd = b.to(dev).detach().requires_grad_(True) if affine else None
    y = layer_norm(xd, wd, bd, 1e-5)
    assert y.dtype == dtype
    y.backward(dy.to(dev))
    lim = 1e-4 if dtype == torch.float32 else 2e-2
    if rows:
        assert max_rel(xd.grad, xr.grad) <= lim, ("dx", max_rel(xd.grad, xr.grad))
    if affine:
        for name, got, ref in (("dw", wd.grad, wr.grad), ("db", bd.grad, br.grad)):
            assert got.dtype == dtype
            if rows:
                assert max_rel(got, ref) <= lim, (name, max_rel(got, ref))
            else:
                assert got.abs().max().item() == 0.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_lm_backward_matches_oracle(dev, dtype):
    """Two-layer LM (d_model 256, 4 heads, d_state 64, vocab 512) at B=2, L=192: the
    gradients of a weighted sum of the logits w.r.t. every parameter that trains in the
    reference, and no gradient for the mixer's parameters."""
    from hdcmamba_amd import HdcMambaLM

    _say("lm backward", dtype)
    torch.manual_seed(0)
    lm = HdcMambaLM(256, 2, 64, 4, vocab_size=512, chunk_size=64)
    for i, blk in enumerate(lm.backbone.layers):
        reinit_block_(blk, seed=30 + i, decays_uniform=True)
    lm = lm.to(dtype).train()
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, 512, (2, 192), generator=g)
    R = torch.randn(2, 192, 512, generator=g)

    sd = {k: v.detach().clone() for k, v in lm.state_dict().items()}
    for i in range(2):  # a training-mode forward refreshes gamma from decay_log first
        sd[f"backbone.layers.{i}.gamma_buf"] = torch.exp(-F.softplus(sd[f"backbone.layers.{i}.decay_log"]))
    for v in sd.values():
        v.requires_grad_(v.is_floating_point())
    ref_logits = oracle.lm_forward(sd, ids, oracle.BlockCfg(256, 64, 4, 64), 2)
    (ref_logits.float() * R).sum().backward()

    lm = lm.to(dev)
    logits = lm(ids.to(dev))
    (logits.float() * R.to(dev)).sum().backward()
    lim = 1e-4 if dtype == torch.float32 else 2e-2
    params = dict(lm.named_parameters())
    trained = ["embedding.weight", "norm_f.weight", "norm_f.bias", "backbone.norm_final.weight",
               "backbone.norm_final.bias"] + [f"backbone.layers.{i}.out_proj.weight" for i in range(2)]
    for name in trained:
        got, ref = params[name].grad, sd[name].grad
        assert got is not None, name
        err = max_rel(got, ref)
        _say(f"  {name}: normwise {err:.2e}")
        assert err <= lim, (name, err)
    for i in range(2):
        for name in ("in_proj.weight", "in_proj.bias", "A_log", "decay_log", "norm.weight", "conv1d.weight",
                     "group_norm.weight"):
            assert params[f"backbone.layers.{i}.{name}"].grad is None, name
