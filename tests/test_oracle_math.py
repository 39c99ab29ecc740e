"""Pins of the oracle that do not depend on the reference's code: library routines,
closed forms, hand-computed known answers and brute force on tiny inputs.  Each group
also shows that a plausible mistake planted in a copy of the oracle fails the pin."""
import math

import pytest
import torch
import torch.nn.functional as F

import oracle

torch.set_default_dtype(torch.float32)


def _g(seed):
    return torch.Generator().manual_seed(seed)


# ----------------------------------------------------------------------------- LN + conv
def _library_norm_conv(x, w, b, cw, cb, eps, halo_beta=True):
    """F.layer_norm then F.conv1d(groups=D); the 3 rows before t=0 are LN of a zero row (= b)."""
    B, L, D = x.shape
    u = F.layer_norm(x, (D,), w, b, eps)
    halo = b.expand(B, 3, D) if halo_beta else torch.zeros(B, 3, D)
    up = torch.cat([halo, u], 1).transpose(1, 2)  # [B, D, L+3]
    return F.conv1d(up, cw.view(D, 1, 4), cb, groups=D).transpose(1, 2)


def test_norm_conv_equals_library_routines():
    g = _g(0)
    x = 3 * torch.randn(2, 33, 48, generator=g) + 1
    w, b = 1 + 0.1 * torch.randn(48, generator=g), 0.3 * torch.randn(48, generator=g)
    cw, cb = 0.4 * torch.randn(48, 4, generator=g), 0.1 * torch.randn(48, generator=g)
    torch.testing.assert_close(oracle.norm_conv(x, w, b, cw, cb, 1e-5), _library_norm_conv(x, w, b, cw, cb, 1e-5),
                               atol=1e-5, rtol=1e-5)
    # planted mistake: a zero halo (nn.Conv1d's own padding) instead of LN(0-row) = b
    wrong = _library_norm_conv(x, w, b, cw, cb, 1e-5, halo_beta=False)
    assert (oracle.norm_conv(x, w, b, cw, cb, 1e-5) - wrong).abs().max() > 1e-2


def test_norm_conv_identity_tap_is_layernorm():
    x = torch.randn(1, 9, 16, generator=_g(1))
    w, b = torch.ones(16), torch.zeros(16)
    cw = torch.zeros(16, 4)
    cw[:, 3] = 1.0
    torch.testing.assert_close(oracle.norm_conv(x, w, b, cw, torch.zeros(16), 1e-5),
                               F.layer_norm(x, (16,), eps=1e-5), atol=1e-6, rtol=1e-6)


# ----------------------------------------------------------------------------- SSM
def _ssm_projs(dt_raw, xs, bs):
    return torch.cat([dt_raw, xs, bs], -1)


def test_ssm_closed_form_constant_inputs():
    """Constant dt, x, b: h_t = u (1 - a^(t+1)) / (1 - a), a = exp(dt*A), u = dt*b*x."""
    ds, L = 3, 50
    dt_raw = torch.tensor([-2.0, 0.0, 1.0]).expand(1, L, ds)
    xs = torch.tensor([0.5, -1.0, 2.0]).expand(1, L, ds)
    bs = torch.tensor([1.5, 0.25, -0.5]).expand(1, L, ds)
    A_log = torch.log(torch.tensor([0.3, 0.9, 1.7]))
    y, h = oracle.ssm_sequential(_ssm_projs(dt_raw, xs, bs), A_log, ds)
    dt = torch.log1p(torch.exp(dt_raw[0, 0]))
    a = torch.exp(-dt * torch.exp(A_log))
    u = dt * bs[0, 0] * xs[0, 0]
    t = torch.arange(L, dtype=torch.float32).view(L, 1)
    closed = u * (1 - a ** (t + 1)) / (1 - a)
    torch.testing.assert_close(y[0], closed, atol=1e-5, rtol=1e-5)
    # planted mistake: the decay applied after the input, h_t = a (h_{t-1} + u)
    bad = a * u * (1 - a ** (t + 1)) / (1 - a)
    assert (y[0] - bad).abs().max() > 1e-2


def test_ssm_sequential_equals_scalar_loop():
    g = _g(2)
    L, ds = 7, 2
    projs = torch.randn(1, L, 3 * ds, generator=g)
    projs[0, 2, 0] = 30.0  # above the softplus threshold
    A_log = torch.tensor([0.1, -0.4])
    y, _ = oracle.ssm_sequential(projs, A_log, ds)
    for d in range(ds):
        h = 0.0
        for t in range(L):
            r = projs[0, t].tolist()
            dt = r[d] if r[d] > 20.0 else math.log(1.0 + math.exp(r[d]))
            h = h * math.exp(dt * -math.exp(A_log[d].item())) + dt * r[2 * ds + d] * r[ds + d]
            assert abs(y[0, t, d].item() - h) <= 1e-5 * max(1.0, abs(h))


@pytest.mark.parametrize("C", [1, 4, 16, 64, 128])
def test_ssm_chunked_is_chunk_invariant(C):
    g = _g(3)
    B, L, ds = 2, 128, 8
    projs = torch.randn(B, L, 3 * ds, generator=g)
    A_log = torch.log(torch.linspace(0.5, 1.5, ds))
    h0 = torch.randn(B, ds, generator=g)
    ys, hs = oracle.ssm_sequential(projs, A_log, ds, h0=h0)
    yc, hc = oracle.ssm_chunked(projs, A_log, ds, C, h0=h0)
    torch.testing.assert_close(yc, ys, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(hc, hs, atol=1e-5, rtol=1e-5)


# ----------------------------------------------------------------------------- slot
def _slot_projs(q, k, v, ds=1, gate=None):
    """Pack per-token q, k, v ([B, L, dm]) into the projs column layout."""
    B, L, dm = q.shape
    lead = torch.zeros(B, L, 3 * ds)
    gate = torch.zeros(B, L, dm) if gate is None else gate
    return torch.cat([lead, q, k, v, gate], -1)


def test_slot_two_token_cross_chunk_rule():
    """Hand-computed: phi(q)=[2, 1.5], phi(k)=[1, 3], v=[1, -2], gamma=0.5.
    C=2 (one chunk):   y1 = 0.5*1.5*1*1 + 1.5*3*(-2) = -8.25
    C=1 (two chunks):  the cross-chunk weight is gamma^(1-0-1) = 1: y1 = 1.5 - 9 = -7.5"""
    q = torch.tensor([1.0, 0.5]).view(1, 2, 1)   # phi = z+1
    k = torch.tensor([0.0, 2.0]).view(1, 2, 1)   # phi(0) = exp(0) = 1, phi(2) = 3
    v = torch.tensor([1.0, -2.0]).view(1, 2, 1)
    projs = _slot_projs(q, k, v)
    gamma = torch.tensor([0.5])
    for fn in (lambda C: oracle.slot_sequential(projs, gamma, 1, 1, 1, C),
               lambda C: oracle.slot_chunked(projs, gamma, 1, 1, 1, C)[0]):
        y2, y1 = fn(2), fn(1)
        assert y2[0, :, 0, 0].tolist() == pytest.approx([2.0, -8.25])
        assert y1[0, :, 0, 0].tolist() == pytest.approx([2.0, -7.5])


def _decayed_attention(projs, gamma, dm, ds, H):
    """Y = (Dec o phi(Q) phi(K)^T) V per head with Dec_ij = gamma^(i-j) for i >= j."""
    B, L, _ = projs.shape
    hd = dm // H
    q = oracle.phi(projs[..., 3 * ds:3 * ds + dm].view(B, L, H, hd)).transpose(1, 2)
    k = oracle.phi(projs[..., 3 * ds + dm:3 * ds + 2 * dm].view(B, L, H, hd)).transpose(1, 2)
    v = projs[..., 3 * ds + 2 * dm:3 * ds + 3 * dm].reshape(B, L, H, hd).transpose(1, 2)
    i = torch.arange(L, dtype=torch.float32)
    e = (i[:, None] - i[None, :])
    dec = torch.where(e >= 0, gamma.view(H, 1, 1) ** e.clamp_min(0), torch.zeros(()))
    return ((q @ k.transpose(-1, -2)) * dec @ v).transpose(1, 2)


def test_slot_single_chunk_is_decayed_attention():
    g = _g(4)
    B, L, dm, ds, H = 2, 24, 8, 2, 2
    projs = 0.5 * torch.randn(B, L, 3 * ds + 4 * dm, generator=g)
    gamma = torch.tensor([0.9, 0.6])
    ref = _decayed_attention(projs, gamma, dm, ds, H)
    torch.testing.assert_close(oracle.slot_sequential(projs, gamma, dm, ds, H, L), ref, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(oracle.slot_chunked(projs, gamma, dm, ds, H, L)[0], ref, atol=1e-5, rtol=1e-5)
    # with several chunks the result must differ (the gamma^-1 cross-chunk factor)
    assert (oracle.slot_chunked(projs, gamma, dm, ds, H, 4)[0] - ref).abs().max() > 1e-3


def test_slot_gamma_one_is_cumulative_sum():
    g = _g(5)
    B, L, dm, ds, H = 1, 16, 4, 1, 1
    projs = 0.5 * torch.randn(B, L, 3 * ds + 4 * dm, generator=g)
    q = oracle.phi(projs[..., 3 * ds:3 * ds + dm])
    k = oracle.phi(projs[..., 3 * ds + dm:3 * ds + 2 * dm])
    v = projs[..., 3 * ds + 2 * dm:3 * ds + 3 * dm]
    S = torch.cumsum(k.unsqueeze(-1) * v.unsqueeze(-2), dim=1)  # [B, L, dk, dv]
    ref = (q.unsqueeze(-2) @ S).squeeze(-2).view(B, L, 1, dm)
    torch.testing.assert_close(oracle.slot_chunked(projs, torch.ones(1), dm, ds, H, L)[0], ref, atol=1e-4, rtol=1e-5)


@pytest.mark.parametrize("C", [1, 2, 8, 16, 32])
def test_slot_chunked_equals_sequential(C):
    g = _g(6)
    B, L, dm, ds, H = 2, 32, 8, 2, 2
    projs = 0.5 * torch.randn(B, L, 3 * ds + 4 * dm, generator=g)
    gamma = torch.tensor([0.93, 0.7])
    y, S = oracle.slot_chunked(projs, gamma, dm, ds, H, C)
    torch.testing.assert_close(y, oracle.slot_sequential(projs, gamma, dm, ds, H, C), atol=1e-4, rtol=1e-5)
    # the carried state is the reference's `running`: sum_j gamma^(L-1-j) phi(k_j)^T v_j
    hd = dm // H
    k = oracle.phi(projs[..., 3 * ds + dm:3 * ds + 2 * dm].view(B, L, H, hd))
    v = projs[..., 3 * ds + 2 * dm:3 * ds + 3 * dm].reshape(B, L, H, hd)
    w = gamma.view(1, H) ** (L - 1 - torch.arange(L, dtype=torch.float32)).view(L, 1)  # [L, H]
    S_ref = torch.einsum("lh,blhk,blhv->bhkv", w, k, v)
    torch.testing.assert_close(S, S_ref, atol=1e-4, rtol=1e-5)


# ----------------------------------------------------------------------------- gate, LN
def test_gnorm_gate_equals_group_norm_and_sigmoid():
    g = _g(7)
    B, L, H, hd = 2, 5, 3, 8
    y = 2 * torch.randn(B, L, H, hd, generator=g) + 0.5
    gate = torch.randn(B, L, H * hd, generator=g)
    w, b = 1 + 0.1 * torch.randn(H * hd, generator=g), 0.1 * torch.randn(H * hd, generator=g)
    ref = F.group_norm(y.reshape(B * L, H * hd, 1), H, w, b, 1e-5).view(B, L, H * hd) * torch.sigmoid(gate)
    torch.testing.assert_close(oracle.gnorm_gate(y, gate, w, b, H), ref, atol=1e-5, rtol=1e-5)
    # planted mistake: statistics over the whole row (nn.GroupNorm over dm) instead of per head
    bad = F.layer_norm(y.reshape(B, L, H * hd), (H * hd,), w, b, 1e-5) * torch.sigmoid(gate)
    assert (oracle.gnorm_gate(y, gate, w, b, H) - bad).abs().max() > 1e-2


@pytest.mark.parametrize("affine", [False, True])
def test_rowln_equals_layer_norm(affine):
    g = _g(8)
    x = 4 * torch.randn(3, 7, 40, generator=g) + 2
    w = 1 + 0.2 * torch.randn(40, generator=g) if affine else None
    b = 0.2 * torch.randn(40, generator=g) if affine else None
    torch.testing.assert_close(oracle.rowln(x, w, b), F.layer_norm(x, (40,), w, b, 1e-5), atol=1e-5, rtol=1e-5)


# ----------------------------------------------------------------------------- faithful maps
def test_faithful_slot_position_kat():
    """The reference's gate kernel reads (l//128, l%128) as (chunk, offset) for any C
    (model.py:288): at C=64 rows 128..191 re-read positions 64..127."""
    pos = oracle.hdcm_oracle.faithful_slot_position(256, 64)
    assert pos[:128].tolist() == list(range(128))
    assert pos[128].item() == 64 and pos[191].item() == 127 and pos[192].item() == 128
    assert pos[255].item() == 191
    assert oracle.hdcm_oracle.faithful_slot_position(256, 128).tolist() == list(range(256))


def test_faithful_gate_index_kat():
    """Gate launch strides (B*L, 4*dm) on a view with true strides (L*P, P) (model.py:377):
    B=2, L=3, dm=4, ds=1 -> element (b=1, l=2, j=1) at 15 + 1*6 + 2*16 + 1 = 54."""
    idx = oracle.hdcm_oracle.faithful_gate_index(2, 3, 4, 1)
    assert idx[1, 2, 1].item() == 54
    assert idx[0, 0, 0].item() == 3 * 1 + 3 * 4
    yi = oracle.hdcm_oracle.faithful_yssm_index(2, 3, 4)
    assert yi[1, 2, 3].item() == 1 * 6 + 2 * 4 + 3


# ----------------------------------------------------------------------------- block
def test_block_intended_fp32_matches_sequential_forms():
    """Block forward built from the chunked oracle pieces equals one built from the brute-force
    sequential forms (fp32, C=4 so that chunk carries occur)."""
    cfg = oracle.BlockCfg(16, 4, 2, 4)
    p = oracle.init_block_params(cfg, generator_seed=3)
    x = torch.randn(1, 12, 16, generator=_g(9))
    y, st = oracle.block_forward(p, x, cfg, return_states=True)
    projs = st["projs"]
    ys, _ = oracle.ssm_sequential(projs, p["A_log"], 4)
    yslot = oracle.slot_sequential(projs, p["gamma_buf"], 16, 4, 2, 4)
    g = oracle.gnorm_gate(yslot, projs[..., 12 + 48:], p["group_norm.weight"], p["group_norm.bias"], 2)
    comb = torch.cat([ys, g], -1)
    ref = x + F.linear(F.layer_norm(comb, (20,)), p["out_proj.weight"])
    torch.testing.assert_close(y, ref, atol=1e-5, rtol=1e-5)


# ----------------------------------------------------------------------------- streaming (prefill -> decode)
def _block_sequential_padded(p, xp, cfg):
    """Block output on an already padded sequence from the brute-force sequential forms
    (library LN+conv, ssm_sequential, slot_sequential with chunk index t // C)."""
    dm, ds, H = cfg.d_model, cfg.d_state, cfg.num_heads
    xc = _library_norm_conv(xp, p["norm.weight"], p["norm.bias"], p["conv1d.weight"].squeeze(1),
                            p["conv1d.bias"], 1e-5)
    projs = F.linear(xc, p["in_proj.weight"], p["in_proj.bias"])
    ys, _ = oracle.ssm_sequential(projs, p["A_log"], ds)
    yslot = oracle.slot_sequential(projs, p["gamma_buf"], dm, ds, H, cfg.chunk_size)
    g = oracle.gnorm_gate(yslot, projs[..., 3 * ds + 3 * dm:], p["group_norm.weight"], p["group_norm.bias"], H)
    comb = torch.cat([ys, g], -1)
    return xp + F.linear(F.layer_norm(comb, (ds + dm,)), p["out_proj.weight"])


def test_stream_with_whole_prefill_is_block_forward():
    cfg = oracle.BlockCfg(16, 4, 2, 4)
    p = oracle.init_block_params(cfg, generator_seed=4)
    x = torch.randn(2, 10, 16, generator=_g(10))
    torch.testing.assert_close(oracle.block_forward_stream(p, x, cfg, 10), oracle.block_forward(p, x, cfg),
                               atol=0, rtol=0)


@pytest.mark.parametrize("n_prefill", [1, 5, 8, 9])
def test_stream_equals_sequential_recurrence(n_prefill):
    """Prefill of n rows then token-by-token continuation: the chunk grid is the prefill's
    (left pad to a multiple of C) and the tail needs no alignment.  Checked against the
    sequential forms on the left-padded sequence, which never see the right padding."""
    cfg = oracle.BlockCfg(16, 4, 2, 4)
    p = oracle.init_block_params(cfg, generator_seed=5)
    x = torch.randn(1, 14, 16, generator=_g(11))
    pad = (4 - n_prefill % 4) % 4
    ref = _block_sequential_padded(p, F.pad(x, (0, 0, pad, 0)), cfg)[:, pad:]
    got = oracle.block_forward_stream(p, x, cfg, n_prefill)
    torch.testing.assert_close(got, ref, atol=1e-5, rtol=1e-5)
    # a plain forward of the whole 14 rows uses a different chunk grid (pad 2): the
    # continuation semantics are not a re-forward unless the grids agree
    if pad != 2:
        assert (oracle.block_forward(p, x, cfg) - got).abs().max() > 1e-4


@pytest.mark.parametrize("n_prefill,C,H", [(8, 4, 2), (5, 4, 2), (1, 4, 4), (9, 3, 2), (6, 1, 2)])
def test_block_step_equals_stream(n_prefill, C, H):
    """block_prefill_state then block_step token by token equals block_forward_stream over
    the same rows: chunk ends inside the steps, left-padded prefills, one-row chunks."""
    cfg = oracle.BlockCfg(16, 4, H, C)
    p = oracle.init_block_params(cfg, generator_seed=6 + C)
    n_dec = 11
    x = torch.randn(2, n_prefill + n_dec, 16, generator=_g(12 + n_prefill))
    ref = oracle.block_forward_stream(p, x, cfg, n_prefill)
    y0, st = oracle.block_prefill_state(p, x[:, :n_prefill], cfg)
    torch.testing.assert_close(y0, ref[:, :n_prefill], atol=1e-5, rtol=1e-5)
    ys = [oracle.block_step(p, x[:, t], st, cfg) for t in range(n_prefill, n_prefill + n_dec)]
    torch.testing.assert_close(torch.stack(ys, 1), ref[:, n_prefill:], atol=1e-4, rtol=1e-4)
    assert st["pos"] == (n_prefill + (C - n_prefill % C) % C + n_dec) % C


def test_block_step_chunk_end_fold_is_needed():
    """Dropping the (gamma^C - gamma^(C-1)) S_prev term of the chunk-end fold (planted in the
    state after the first chunk end) makes the continuation miss the stream form."""
    cfg = oracle.BlockCfg(16, 4, 2, 4)
    p = oracle.init_block_params(cfg, generator_seed=21)
    x = torch.randn(2, 8 + 9, 16, generator=_g(22))
    ref = oracle.block_forward_stream(p, x, cfg, 8)
    _, st = oracle.block_prefill_state(p, x[:, :8], cfg)
    g = p["gamma_buf"].float().view(1, 2, 1, 1)
    ys, planted = [], False
    for t in range(8, 17):
        c, s_prev = st["pos"], st["S_prev"].clone()
        ys.append(oracle.block_step(p, x[:, t], st, cfg))
        if c == 3 and not planted:
            st["S_prev"] = st["S_prev"] - (g ** 4 - g ** 3) * s_prev
            planted = True
    assert planted
    assert (torch.stack(ys, 1) - ref[:, 8:]).abs().max() > 1e-3


# ----------------------------------------------------------------------------- norm_conv gradients
def _norm_conv_library(x, w, b, cw, cb, eps):
    """LayerNorm then depthwise conv1d through PyTorch's own modules, the three rows before
    the sequence start being the LayerNorm of a zero row (= b)."""
    B, L, D = x.shape
    u = torch.nn.functional.layer_norm(x, (D,), w, b, eps)
    up = torch.cat([b.expand(B, 3, D), u], 1).transpose(1, 2)
    return torch.nn.functional.conv1d(up, cw.unsqueeze(1), cb, groups=D).transpose(1, 2)


def _grad_inputs(seed, B=2, L=7, D=16, beta=0.3):
    g = torch.Generator().manual_seed(seed)
    t = lambda *s, sc=1.0, off=0.0: (sc * torch.randn(*s, generator=g) + off).requires_grad_()
    return [t(B, L, D, sc=2.0, off=0.5), t(D, sc=0.2, off=1.0), t(D, sc=beta), t(D, 4, sc=0.5), t(D, sc=0.1)]


def test_norm_conv_gradients_equal_library_autograd():
    """Gradients of the oracle's LN+conv (all five inputs) equal those PyTorch's layer_norm
    and conv1d backward kernels give for the same forward, LN-bias halo included."""
    ins = _grad_inputs(0)
    go = torch.randn(2, 7, 16, generator=torch.Generator().manual_seed(1))
    g_or = torch.autograd.grad(oracle.norm_conv(*ins, 1e-5), ins, go)
    g_lib = torch.autograd.grad(_norm_conv_library(*ins, 1e-5), ins, go)
    for a, b, name in zip(g_or, g_lib, ["x", "ln_w", "ln_b", "conv_w", "conv_b"]):
        torch.testing.assert_close(a, b, atol=1e-5, rtol=1e-5, msg=name)


def test_norm_conv_gradients_finite_differences():
    """The oracle's gradients against central differences (fp32, step 1e-2)."""
    ins = [t.detach().double().requires_grad_() for t in _grad_inputs(2, B=1, L=5, D=8)]
    fn = lambda *a: oracle.norm_conv(*[t.float() for t in a], 1e-5).double()
    assert torch.autograd.gradcheck(fn, ins, eps=1e-2, atol=2e-3, rtol=2e-3)


def test_norm_conv_bias_gradient_includes_the_halo():
    """d ln_b collects the conv taps that read the LayerNorm-of-zero rows before the start:
    with a gradient on out[0] only, d ln_b = B (w0 + w1 + w2) from the three halo rows plus
    B w3 from the b term of u[0].  A backward that drops the halo (as the reference kernel
    does) gets B w3 only."""
    ins = _grad_inputs(3)
    go = torch.zeros(2, 7, 16)
    go[:, 0] = 1.0  # only out[0] matters: u[-3], u[-2], u[-1] (= b) and u[0]
    grads = torch.autograd.grad(oracle.norm_conv(*ins, 1e-5), ins, go)
    cw = ins[3].detach()
    # d out[0] / d b = sum of the three halo taps + the tap on u[0] (whose b term is 1)
    want = 2 * (cw[:, 0] + cw[:, 1] + cw[:, 2] + cw[:, 3])
    torch.testing.assert_close(grads[2], want, atol=1e-5, rtol=1e-5)


def test_oracle_training_gradients_follow_the_reference():
    """The reference's mixer kernels have no autograd (model.py:340-384): through the oracle
    block, out_proj and the input get gradients and the mixer's parameters none, unless
    mixer_grad asks for the full derivative (then in_proj gets one too)."""
    cfg = oracle.BlockCfg(64, 16, 2, 16)
    p = oracle.init_block_params(cfg, generator_seed=3)
    for mixer_grad in (False, True):
        q = {k: v.detach().clone().requires_grad_(v.is_floating_point()) for k, v in p.items()}
        x = torch.randn(1, 32, 64, generator=torch.Generator().manual_seed(4)).requires_grad_(True)
        oracle.block_forward(q, x, cfg, mixer_grad=mixer_grad).square().sum().backward()
        assert q["out_proj.weight"].grad is not None and x.grad is not None
        assert (q["in_proj.weight"].grad is not None) == mixer_grad
        assert (q["norm.weight"].grad is not None) == mixer_grad


@pytest.mark.parametrize("C", [4, 8, 32])
def test_attend_chunked_equals_brute_force(C):
    """The chunked slot recurrence on arbitrary (signed) featured q/k equals the brute-force
    double loop with the gamma^(t-j) / gamma^(t-j-1) weights."""
    g = torch.Generator().manual_seed(C)
    B, L, H, hk, hd = 2, 32, 3, 8, 5
    qf, kf = torch.randn(B, L, H, hk, generator=g), torch.randn(B, L, H, hk, generator=g)
    v = torch.randn(B, L, H, hd, generator=g)
    gamma = torch.tensor([0.9, 0.6, 1.0])
    y, _ = oracle.attend_chunked(qf, kf, v, gamma, C)
    ref = oracle.attend_sequential(qf, kf, v, gamma, C)
    torch.testing.assert_close(y, ref, atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("C", [4, 16])
def test_attend_gradients_are_attend_passes(C):
    """The three gradient contractions of the slot recurrence are the recurrence itself
    (autograd through the brute force pins them): dq = attend(dy, v, k) forward in time,
    dv = attend(k, q, dy) and dk = attend(v, dy, q) backward in time (L a multiple of C,
    so the chunk grid maps onto itself)."""
    g = torch.Generator().manual_seed(100 + C)
    B, L, H, hk = 1, 32, 2, 6
    qf = torch.randn(B, L, H, hk, generator=g).requires_grad_(True)
    kf = torch.randn(B, L, H, hk, generator=g).requires_grad_(True)
    v = torch.randn(B, L, H, hk, generator=g).requires_grad_(True)
    dy = torch.randn(B, L, H, hk, generator=g)
    gamma = torch.tensor([0.8, 0.95])
    (oracle.attend_sequential(qf, kf, v, gamma, C) * dy).sum().backward()
    fl = lambda t: t.detach().flip(1)
    dq = oracle.attend_chunked(dy, v.detach(), kf.detach(), gamma, C)[0]
    dv = oracle.attend_chunked(fl(kf), fl(qf), fl(dy), gamma, C)[0].flip(1)
    dk = oracle.attend_chunked(fl(v), fl(dy), fl(qf), gamma, C)[0].flip(1)
    for name, got, ref in (("dq", dq, qf.grad), ("dv", dv, v.grad), ("dk", dk, kf.grad)):
        torch.testing.assert_close(got, ref, atol=1e-4, rtol=1e-4, msg=name)


# ----------------------------------------------------------------------------- LM wrapper
def test_lm_forward_hidden_and_positions():
    """lm_forward's head input (return_hidden) is norm_f over the blocks and norm_final composed
    by hand, and the logits at chosen positions are the tied head applied to it there."""
    cfg = oracle.BlockCfg(16, 4, 2, 4)
    V, n_layers = 40, 2
    sd = {}
    for i in range(n_layers):
        for k, v in oracle.init_block_params(cfg, generator_seed=20 + i).items():
            sd[f"backbone.layers.{i}.{k}"] = v
    g = _g(21)
    sd["backbone.norm_final.weight"] = 1 + 0.1 * torch.randn(16, generator=g)
    sd["backbone.norm_final.bias"] = 0.1 * torch.randn(16, generator=g)
    sd["norm_f.weight"] = 1 + 0.1 * torch.randn(16, generator=g)
    sd["norm_f.bias"] = 0.1 * torch.randn(16, generator=g)
    sd["embedding.weight"] = torch.randn(V, 16, generator=g)
    ids = torch.randint(0, V, (2, 10), generator=g)
    pos = [0, 3, 9]
    logits, h = oracle.lm_forward(sd, ids, cfg, n_layers, positions=pos, return_hidden=True)
    x = F.embedding(ids, sd["embedding.weight"])
    for i in range(n_layers):
        x = oracle.block_forward({k[len(f"backbone.layers.{i}."):]: v for k, v in sd.items()
                                  if k.startswith(f"backbone.layers.{i}.")}, x, cfg)
    x = F.layer_norm(x, (16,), sd["backbone.norm_final.weight"], sd["backbone.norm_final.bias"], 1e-5)
    want_h = F.layer_norm(x, (16,), sd["norm_f.weight"], sd["norm_f.bias"], 1e-5)
    torch.testing.assert_close(h, want_h, atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(logits, F.linear(want_h[:, pos], sd["embedding.weight"]), atol=1e-5, rtol=1e-5)
    assert torch.equal(logits, oracle.lm_forward(sd, ids, cfg, n_layers, positions=pos))
