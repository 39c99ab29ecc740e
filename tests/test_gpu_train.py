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


def test_block_and_model_sum_backward(dev):
    """``model(x).sum().backward()`` in training mode, as the reference's benchmark times the
    backward (benchmark.py:196-205), for one block and for a two-layer model (bf16)."""
    from hdcmamba_amd import HdcMamba9v3Block, HdcMamba9v3Model

    _say("block/model sum backward")
    cfg = oracle.BlockCfg(256, 64, 4, 64)
    torch.manual_seed(1)
    blk = reinit_block_(HdcMamba9v3Block(256, 64, 4, 64), seed=41, decays_uniform=True).to(torch.bfloat16).train()
    x = torch.randn(2, 200, 256, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    sd = {k: v.detach().clone() for k, v in blk.state_dict().items()}
    sd["gamma_buf"] = torch.exp(-F.softplus(sd["decay_log"]))
    for v in sd.values():
        v.requires_grad_(v.is_floating_point())
    xr = x.clone().requires_grad_(True)
    oracle.block_forward(sd, xr, cfg).float().sum().backward()
    blk = blk.to(dev)
    xd = x.to(dev).requires_grad_(True)
    y, none = blk(xd)
    assert none is None
    y.float().sum().backward()
    assert max_rel(xd.grad, xr.grad) <= 2e-2
    assert max_rel(blk.out_proj.weight.grad, sd["out_proj.weight"].grad) <= 2e-2
    assert blk.in_proj.weight.grad is None

    m = HdcMamba9v3Model(256, 2, 64, 32, num_heads=4, chunk_size=64).to(torch.bfloat16).to(dev).train()
    out = m(x.to(dev))
    out.sum().backward()
    assert m.norm_final.weight.grad is not None
    assert all(layer.out_proj.weight.grad is not None for layer in m.layers)


def test_lm_step_under_autocast(dev):
    """One optimiser step of the LM in bf16 under autocast with a cross-entropy loss, as the
    reference's training loop runs it (train_fineweb.py:161-179): finite loss and gradient
    norm, and the step changes exactly the parameters that have gradients."""
    from hdcmamba_amd import HdcMambaLM

    _say("lm step autocast")
    torch.manual_seed(3)
    lm = HdcMambaLM(256, 2, 64, 4, vocab_size=512, chunk_size=64).to(dev).to(torch.bfloat16).train()
    opt = torch.optim.AdamW(lm.parameters(), lr=0.05)  # steps larger than a bf16 ulp of 1.0
    ids = torch.randint(0, 512, (2, 129), device=dev)
    before = {k: v.detach().clone() for k, v in lm.named_parameters()}
    with torch.amp.autocast("cuda", dtype=torch.bfloat16):
        logits = lm(ids[:, :-1])
        loss = F.cross_entropy(logits.reshape(-1, 512).float(), ids[:, 1:].reshape(-1))
    loss.backward()
    norm = torch.nn.utils.clip_grad_norm_(lm.parameters(), max_norm=1.0)
    assert torch.isfinite(loss) and torch.isfinite(norm)
    opt.step()
    for k, v in lm.named_parameters():
        changed = not torch.equal(v.detach(), before[k])
        assert changed == (v.grad is not None), k


# ----------------------------------------------------------------- differentiable mixer
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ssm_backward(dev, dtype):
    """d dt_raw, d x, d b and d A_log of the scan against autograd through the oracle's
    sequential recurrence (fp32, on the same rounded inputs); some dt_raw above the
    softplus threshold 20."""
    from hdcmamba_amd import _ops

    _say("ssm bwd", dtype)
    g = torch.Generator().manual_seed(5)
    B, L, ds = 2, 300, 64
    projs = (0.5 * torch.randn(B, L, 3 * ds + 8, generator=g)).to(dtype)
    projs[0, 7, 3] = 25.0
    A_log = torch.log(torch.linspace(0.5, 2.0, ds)).to(dtype)
    gy = torch.randn(B, L, ds, generator=g).to(dtype)
    pr = projs.float().clone().requires_grad_(True)
    ar = A_log.float().clone().requires_grad_(True)
    y, _ = oracle.ssm_sequential(pr, ar, ds)
    (y * gy.float()).sum().backward()
    pd = projs.to(dev)
    h = torch.empty(B, L, ds, device=dev, dtype=dtype)
    _ops.ssm(pd, A_log.to(dev), ds, h)
    dprojs = torch.zeros(B, L, 3 * ds + 8, device=dev, dtype=dtype)
    dA = _ops.ssm_bwd(pd, A_log.to(dev), ds, h, gy.to(dev), dprojs)
    lim = 1e-4 if dtype == torch.float32 else 2e-2
    for name, got, ref in (("d dt_raw", dprojs[..., :ds], pr.grad[..., :ds]),
                           ("d x", dprojs[..., ds:2 * ds], pr.grad[..., ds:2 * ds]),
                           ("d b", dprojs[..., 2 * ds:3 * ds], pr.grad[..., 2 * ds:3 * ds]),
                           ("d A_log", dA, ar.grad)):
        err = max_rel(got, ref)
        _say(f"  {name}: {err:.2e}")
        assert err <= lim, (name, err)


@pytest.mark.parametrize("dtype,H,dm,B,L", [(torch.float32, 4, 256, 2, 100), (torch.bfloat16, 4, 256, 2, 100),
                                            (torch.bfloat16, 8, 256, 2, 100), (torch.float32, 2, 256, 2, 100),
                                            (torch.bfloat16, 8, 768, 2, 100), (torch.float32, 8, 768, 1, 70),
                                            (torch.bfloat16, 4, 512, 1, 2600), (torch.float32, 16, 1024, 1, 2051),
                                            (torch.bfloat16, 16, 768, 2, 90), (torch.float32, 16, 256, 2, 90),
                                            (torch.bfloat16, 8, 640, 1, 70)])
def test_gnorm_gate_backward(dev, dtype, H, dm, B, L):
    """dy, d gate, d gn_w, d gn_b of the per-token GroupNorm + gate against autograd through
    the oracle: head dims 64, 32, 128 and 16 (row-stripe kernel; one partial stripe at dm 256,
    more tokens than the 2048 waves at L 2600 and 2051) and 96, 48, 80 (per-head kernel)."""
    from hdcmamba_amd import _ops

    _say("gnorm gate bwd", dtype, H, dm, B, L)
    g = torch.Generator().manual_seed(H + L)
    y = (2 * torch.randn(B, L, dm, generator=g) + 0.5).to(dtype)
    gate = torch.randn(B, L, dm, generator=g).to(dtype)
    w = (1 + 0.2 * torch.randn(dm, generator=g)).to(dtype)
    b = (0.1 * torch.randn(dm, generator=g)).to(dtype)
    do = torch.randn(B, L, dm, generator=g).to(dtype)
    yr, gr, wr, br = (t.float().clone().requires_grad_(True) for t in (y, gate, w, b))
    out = oracle.gnorm_gate(yr.view(B, L, H, dm // H), gr, wr, br, H)
    (out * do.float()).sum().backward()
    dy = torch.empty(B, L, dm, device=dev, dtype=dtype)
    dg = torch.empty(B, L, dm, device=dev, dtype=dtype)
    dgw, dgb = _ops.gnorm_gate_bwd(y.to(dev), gate.to(dev), w.to(dev), b.to(dev), 1e-5, do.to(dev), H, dy, dg)
    lim = 1e-4 if dtype == torch.float32 else 2e-2
    for name, got, ref in (("dy", dy, yr.grad), ("d gate", dg, gr.grad), ("d gn_w", dgw, wr.grad),
                           ("d gn_b", dgb, br.grad)):
        err = max_rel(got, ref)
        _say(f"  {name}: {err:.2e}")
        assert err <= lim, (name, err)


@pytest.mark.parametrize("dtype,L,dm,H,C", [(torch.float32, 192, 256, 4, 64), (torch.bfloat16, 192, 256, 4, 64),
                                            (torch.float32, 100, 256, 4, 64),
                                            (torch.bfloat16, 144, 384, 8, 48),   # hd 48, C 48
                                            (torch.float32, 160, 320, 4, 80)])  # hd 80, C 80
def test_differentiable_mixer_block(dev, dtype, L, dm, H, C):
    """A block with differentiable_mixer: gradients of every parameter but decay_log and of
    the input against autograd through the oracle block with mixer_grad (the full derivative
    of the intended forward, gamma held constant)."""
    from hdcmamba_amd import HdcMamba9v3Block

    _say("differentiable mixer", dtype, L, dm, H, C)
    cfg = oracle.BlockCfg(dm, 64, H, C)
    torch.manual_seed(2)
    blk = reinit_block_(HdcMamba9v3Block(dm, 64, H, C, differentiable_mixer=True), seed=51,
                        decays_uniform=True).to(dtype).train()
    with torch.no_grad():  # non-trivial LayerNorm / GroupNorm affine parameters
        for t in (blk.norm.weight, blk.group_norm.weight):
            t.add_(0.1 * torch.randn(t.shape, generator=torch.Generator().manual_seed(52)).to(dtype))
        for t in (blk.norm.bias, blk.group_norm.bias):
            t.add_(0.05 * torch.randn(t.shape, generator=torch.Generator().manual_seed(53)).to(dtype))
    x = torch.randn(2, L, dm, generator=torch.Generator().manual_seed(54)).to(dtype)
    R = torch.randn(2, L, dm, generator=torch.Generator().manual_seed(55))
    sd = {k: v.detach().clone() for k, v in blk.state_dict().items()}
    sd["gamma_buf"] = torch.exp(-F.softplus(sd["decay_log"]))
    for v in sd.values():
        v.requires_grad_(v.is_floating_point())
    xr = x.clone().requires_grad_(True)
    (oracle.block_forward(sd, xr, cfg, mixer_grad=True).float() * R).sum().backward()
    blk = blk.to(dev)
    xd = x.to(dev).requires_grad_(True)
    y, _ = blk(xd)
    (y.float() * R.to(dev)).sum().backward()
    lim = 1e-4 if dtype == torch.float32 else 2e-2
    params = dict(blk.named_parameters())
    names = ["in_proj.weight", "in_proj.bias", "A_log", "group_norm.weight", "group_norm.bias", "norm.weight",
             "norm.bias", "conv1d.weight", "conv1d.bias", "out_proj.weight"]
    for name in names:
        got, ref = params[name].grad, sd[name].grad
        assert got is not None, name
        err = max_rel(got, ref)
        _say(f"  {name}: {err:.2e}")
        assert err <= lim, (name, err)
    err = max_rel(xd.grad, xr.grad)
    _say(f"  x: {err:.2e}")
    assert err <= lim
    assert params["decay_log"].grad is None
