"""Kernel-level parity of the HIP path against the CPU oracle (same seeded inputs).

Tolerances: fp32 max-abs/rel 1e-4, bf16 2e-2 (assert_close atol=rtol).
"""
import pytest
import torch

import oracle
from hdcmamba_amd import _ops
from cfgs import assert_close, slot_inputs, ssm_inputs

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16]


def _say(*a):
    print(*a, flush=True)


# ----------------------------------------------------------------------------- norm_conv
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("D,L", [(256, 1), (256, 5), (768, 100), (1024, 257), (2048, 64), (3072, 37)])
def test_norm_conv(dev, dtype, D, L):
    _say("norm_conv", dtype, D, L)
    g = torch.Generator().manual_seed(D + L)
    B = 2
    x = (3 * torch.randn(B, L, D, generator=g) + 0.5).to(dtype)
    ln_w = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype)
    ln_b = (0.1 * torch.randn(D, generator=g)).to(dtype)
    cw = (0.3 * torch.randn(D, 4, generator=g)).to(dtype)
    cb = (0.1 * torch.randn(D, generator=g)).to(dtype)
    out = _ops.norm_conv(x.to(dev), ln_w.to(dev), ln_b.to(dev), cw.to(dev), cb.to(dev), 1e-5)
    ref = oracle.norm_conv(x, ln_w, ln_b, cw, cb, 1e-5)
    assert_close(out, ref, dtype, "norm_conv")


@pytest.mark.parametrize("D,L", [(2560, 50), (4096, 37), (6144, 19)])
def test_norm_conv_wide_rows_bf16(dev, D, L):
    """bf16 rows wider than 32 columns per lane take the one-row-at-a-time path (up to the 6144
    limit); L not a multiple of the 16-row run covers its partial last run."""
    _say("norm_conv wide", D, L)
    test_norm_conv(dev, torch.bfloat16, D, L)


@pytest.mark.parametrize("D,L", [(4096, 33), (6144, 18)])
def test_norm_conv_backward_wide_bf16(dev, D, L):
    """bf16 rows up to the forward's 6144 columns through the shared-row backward kernel."""
    test_norm_conv_backward(dev, torch.bfloat16, 1, L, D)


def test_norm_conv_batch_strided(dev):
    """A batch-strided view (rows 3.. of a longer buffer) is read through its strides."""
    g = torch.Generator().manual_seed(7)
    D = 512
    full = torch.randn(3, 40, D, generator=g)
    x = full[:, 3:, :]
    p = [torch.ones(D), torch.zeros(D) + 0.2, 0.3 * torch.randn(D, 4, generator=g), torch.zeros(D)]
    out = _ops.norm_conv(full.to(dev)[:, 3:, :], *[t.to(dev) for t in p], 1e-5)
    ref = oracle.norm_conv(x.contiguous(), *p, 1e-5)
    assert_close(out, ref, torch.float32, "norm_conv strided")


# ----------------------------------------------------------------------------- rowln
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,W", [(37, 320), (111, 1024), (5000, 768), (8192, 1024), (33, 2048)])
def test_rowln2_equals_two_passes(dev, dtype, rows, W):
    """Two affine LayerNorms in one pass (norm_final then the LM's norm_f) equal two single
    passes bit for bit, also in place; and the oracle's two row LayerNorms within tolerance.
    5000 and 8192 rows take the four-rows-per-wave path, the others one row per workgroup."""
    _say("rowln2", dtype, rows, W)
    g = torch.Generator().manual_seed(rows + W)
    x = (3 * torch.randn(rows, W, generator=g) + 1).to(dtype)
    p = [(1 + 0.2 * torch.randn(W, generator=g)).to(dtype), (0.3 * torch.randn(W, generator=g)).to(dtype),
         (1 + 0.2 * torch.randn(W, generator=g)).to(dtype), (0.3 * torch.randn(W, generator=g)).to(dtype)]
    xd = x.to(dev)
    w1, b1, w2, b2 = [t.to(dev) for t in p]
    two = _ops.layer_norm(_ops.layer_norm(xd, w1, b1, 1e-5), w2, b2, 1e-6)
    one = _ops.layer_norm2(xd, w1, b1, 1e-5, w2, b2, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(one, two)
    _ops.layer_norm2(xd, w1, b1, 1e-5, w2, b2, 1e-6, out=xd)
    torch.cuda.synchronize()
    assert torch.equal(xd, two)
    ref = oracle.rowln(oracle.rowln(x, p[0], p[1], 1e-5).to(dtype), p[2], p[3], 1e-6)
    assert_close(one, ref, dtype, "rowln2")


def test_rowln2_rejects_rows_past_its_width(dev):
    """Rows wider than 512 16-byte groups are refused (the model runs two passes there)."""
    x = torch.zeros(4, 4104, device=dev, dtype=torch.bfloat16)
    w = torch.ones(4104, device=dev, dtype=torch.bfloat16)
    assert not _ops.layer_norm2_ok(x) and _ops.layer_norm2_ok(x[:, :4096])
    with pytest.raises(RuntimeError):
        _ops.layer_norm2(x, w, w, 1e-5, w, w, 1e-5)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("W", [320, 832, 1152, 2176])
@pytest.mark.parametrize("affine", [False, True])
def test_rowln(dev, dtype, W, affine):
    _say("rowln", dtype, W, affine)
    g = torch.Generator().manual_seed(W)
    x = (5 * torch.randn(3, 37, W, generator=g) + 2).to(dtype)
    w = (1 + 0.2 * torch.randn(W, generator=g)).to(dtype) if affine else None
    b = (0.2 * torch.randn(W, generator=g)).to(dtype) if affine else None
    xd = x.to(dev)
    out = _ops.layer_norm(xd, w.to(dev) if affine else None, b.to(dev) if affine else None, 1e-5)
    ref = oracle.rowln(x, w, b, 1e-5)
    assert_close(out, ref, dtype, "rowln")
    _ops.layer_norm(xd, w.to(dev) if affine else None, b.to(dev) if affine else None, 1e-5, out=xd)
    assert_close(xd, ref, dtype, "rowln in place")


# ----------------------------------------------------------------------------- ssm
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("ds,B,L", [(64, 1, 256), (128, 2, 200), (64, 3, 1000), (32, 2, 700), (192, 1, 3000),
                                    (40, 2, 1500), (128, 1, 32768), (64, 1, 70000)])
def test_ssm(dev, dtype, ds, B, L):
    """ds=40: a partial 32-channel block; L=70000: 137 tiles of 512 rows, three look-back
    windows of 64 tiles."""
    _say("ssm", dtype, ds, B, L)
    projs, A_log = ssm_inputs(B, L, ds, dtype)
    buf = torch.zeros(B, L, ds + 16, device=dev, dtype=dtype)
    hf = torch.empty(B, ds, device=dev)
    _ops.ssm(projs.to(dev), A_log.to(dev), ds, buf[..., :ds], h_final=hf)
    y_ref, h_ref = oracle.ssm_sequential(projs, A_log, ds)
    assert_close(buf[..., :ds], y_ref.to(dtype), dtype, "ssm y")
    assert_close(hf, h_ref, dtype, "ssm h_final")
    assert buf[..., ds:].abs().max().item() == 0.0


@pytest.mark.parametrize("dtype", DTYPES)
def test_ssm_totals_computed_for_their_owners(dev, dtype):
    """With no polling budget a workgroup that finds an earlier tile's total missing computes
    it itself and publishes it for its owner; the outputs are bit-identical to the default
    (the same code computes every total), with a start state and the final state.  L=40000:
    79 tiles, so the computed totals span two look-back windows."""
    print("ssm forced fallback", dtype, flush=True)
    ds, B, L = 128, 2, 40000
    projs, A_log = ssm_inputs(B, L, ds, dtype)
    pd, ad = projs.to(dev), A_log.to(dev)
    h0 = torch.randn(B, ds, generator=torch.Generator().manual_seed(3)).to(dev)
    outs = []
    for spin in (None, 0):
        y = torch.empty(B, L, ds, device=dev, dtype=dtype)
        hf = torch.empty(B, ds, device=dev)
        if spin is None:
            _ops.ssm(pd, ad, ds, y, h0=h0, h_final=hf)
        else:
            with _ops.option("ssm_spin_rounds", spin):
                _ops.ssm(pd, ad, ds, y, h0=h0, h_final=hf)
        torch.cuda.synchronize()
        outs.append((y, hf))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])
    y_ref, h_ref = oracle.ssm_sequential(projs, A_log, ds, h0=h0.cpu())
    assert_close(outs[1][0], y_ref.to(dtype), dtype, "ssm y (fallback)")
    assert_close(outs[1][1], h_ref, dtype, "ssm h_final (fallback)")


def test_ssm_workspace_reused_across_shapes(dev):
    """One workspace serves calls of different shapes in turn: every call's totals carry that
    call's tag, so words left by an earlier call of another shape are never taken for its."""
    dtype = torch.bfloat16
    for B, L, ds in ((2, 4000, 128), (1, 700, 64), (3, 2500, 192), (2, 4000, 128)):
        print("ssm reuse", B, L, ds, flush=True)
        projs, A_log = ssm_inputs(B, L, ds, dtype, seed=B * L + ds)
        y = torch.empty(B, L, ds, device=dev, dtype=dtype)
        hf = torch.empty(B, ds, device=dev)
        _ops.ssm(projs.to(dev), A_log.to(dev), ds, y, h_final=hf)
        y_ref, h_ref = oracle.ssm_sequential(projs, A_log, ds)
        assert_close(y, y_ref.to(dtype), dtype, f"ssm y {B},{L},{ds}")
        assert_close(hf, h_ref, dtype, f"ssm h_final {B},{L},{ds}")


def test_ssm_h0_continuation(dev):
    """Running [0,L/2) then [L/2,L) with the carried state equals one run."""
    ds, B, L = 64, 2, 512
    projs, A_log = ssm_inputs(B, L, ds, torch.float32)
    pd, ad = projs.to(dev), A_log.to(dev)
    y = torch.empty(B, L, ds, device=dev)
    _ops.ssm(pd, ad, ds, y)
    y1 = torch.empty(B, L // 2, ds, device=dev)
    y2 = torch.empty(B, L // 2, ds, device=dev)
    h = torch.empty(B, ds, device=dev)
    _ops.ssm(pd[:, :L // 2].contiguous(), ad, ds, y1, h_final=h)
    _ops.ssm(pd[:, L // 2:].contiguous(), ad, ds, y2, h0=h)
    assert_close(torch.cat([y1, y2], 1), y, torch.float32, "ssm split")


# ----------------------------------------------------------------------------- slot + gate
SLOT_CASES = [
    # (dtype, B, L, dm, H, C)
    (torch.float32, 1, 256, 256, 8, 64),     # hd 32
    (torch.float32, 2, 192, 512, 8, 64),     # hd 64
    (torch.float32, 1, 256, 768, 8, 64),     # hd 96
    (torch.float32, 1, 256, 256, 4, 32),     # C = TC
    (torch.float32, 1, 256, 256, 4, 16),     # C < TC: cross-chunk weights inside a tile
    (torch.float32, 1, 512, 256, 4, 128),    # C > TC: carried within-chunk state
    (torch.float32, 1, 512, 256, 4, 256),
    (torch.bfloat16, 1, 256, 256, 8, 64),
    (torch.bfloat16, 2, 512, 1024, 16, 64),  # hd 64
    (torch.bfloat16, 1, 256, 768, 8, 64),    # hd 96
    (torch.bfloat16, 1, 512, 512, 8, 32),
    (torch.bfloat16, 1, 512, 512, 8, 256),
    (torch.bfloat16, 2, 96, 256, 4, 32),     # last row tile half full (32 of 64 rows)
    (torch.float32, 1, 256, 512, 4, 64),     # hd 128
    (torch.float32, 1, 256, 512, 4, 16),     # hd 128, C < TC
    (torch.bfloat16, 2, 320, 1024, 8, 64),   # hd 128 (d_model 1024 with the default 8 heads)
    (torch.bfloat16, 1, 512, 512, 4, 128),   # hd 128, C > TC
    # head dims that are multiples of 16 but not of 32 (zero-padded contraction columns)
    (torch.bfloat16, 1, 256, 256, 16, 64),   # hd 16
    (torch.float32, 2, 192, 256, 16, 64),    # hd 16
    (torch.bfloat16, 2, 320, 768, 16, 64),   # hd 48 (d_model 768 with 16 heads)
    (torch.float32, 1, 256, 384, 8, 32),     # hd 48
    (torch.bfloat16, 1, 384, 640, 8, 128),   # hd 80, C > TC
    (torch.float32, 1, 256, 320, 4, 16),     # hd 80, C < TC
    (torch.bfloat16, 1, 256, 896, 8, 64),    # hd 112
    # chunks that neither divide the row tile nor are multiples of it (chunk-confined tiles)
    (torch.bfloat16, 1, 288, 256, 4, 48),    # C 48 < TC: one chunk per tile, 16 rows idle
    (torch.bfloat16, 2, 384, 512, 8, 96),    # C 96 > TC: tiles of 64 + 32 rows per chunk
    (torch.float32, 1, 240, 256, 4, 48),     # fp32 (TC 32): tiles of 32 + 16 rows per chunk
    (torch.float32, 1, 240, 256, 4, 24),     # fp32 C 24 < TC
    (torch.bfloat16, 1, 250, 256, 4, 50),    # C not a multiple of 16
    (torch.bfloat16, 1, 1000, 256, 4, 100),  # several segments of whole chunks
]


def _run_slot(dev, projs, gamma, gn_w, gn_b, dm, ds, H, C, S0=None):
    B, L, _ = projs.shape
    pd = projs.to(dev)
    hd = dm // H
    out = torch.zeros(B, L, ds + dm, device=dev, dtype=projs.dtype)
    ws = _ops.slot_workspace(pd, dm, H, C)
    _ops.slot_state(pd, 3 * ds, gamma.to(dev), dm, H, C, ws, S0=S0)
    sf = torch.empty(B, H, hd, hd, device=dev)
    _ops.slot_gate(pd, 3 * ds, gamma.to(dev), gn_w.to(dev), gn_b.to(dev), 1e-5, ws, out, ds, dm, H, C,
                   S_final=sf)
    return out, sf


@pytest.mark.parametrize("dtype,B,L,dm,H,C", SLOT_CASES)
def test_slot_gate(dev, dtype, B, L, dm, H, C):
    _say("slot_gate", dtype, B, L, dm, H, C)
    ds = 64
    projs, gamma, gn_w, gn_b = slot_inputs(B, L, dm, ds, H, dtype, seed=L + dm + C)
    out, sf = _run_slot(dev, projs, gamma, gn_w, gn_b, dm, ds, H, C)
    y, S = oracle.slot_chunked(projs, gamma, dm, ds, H, C, dtype)
    ref = oracle.gnorm_gate(y, projs[..., 3 * ds + 3 * dm:], gn_w, gn_b, H).to(dtype)
    assert_close(out[..., ds:], ref, dtype, "slot+gate")
    assert out[..., :ds].abs().max().item() == 0.0
    assert_close(sf / S.abs().max(), S / S.abs().max(), dtype, "slot S_final")


@pytest.mark.parametrize("out_col", [4, 8])
def test_slot_gate_output_alignment(dev, out_col):
    """bf16 outputs whose rows are only 8-byte aligned take the 8-byte store path; 16-byte
    aligned ones the exchanged 16-byte path.  Both match the oracle."""
    _say("slot_gate out_col", out_col)
    dm, ds, H, C, B, L = 512, 64, 8, 64, 1, 320
    dtype = torch.bfloat16
    projs, gamma, gn_w, gn_b = slot_inputs(B, L, dm, ds, H, dtype, seed=out_col)
    pd = projs.to(dev)
    out = torch.zeros(B, L, out_col + dm, device=dev, dtype=dtype)
    ws = _ops.slot_workspace(pd, dm, H, C)
    _ops.slot_state(pd, 3 * ds, gamma.to(dev), dm, H, C, ws)
    _ops.slot_gate(pd, 3 * ds, gamma.to(dev), gn_w.to(dev), gn_b.to(dev), 1e-5, ws, out, out_col, dm, H, C)
    y, _ = oracle.slot_chunked(projs, gamma, dm, ds, H, C, dtype)
    ref = oracle.gnorm_gate(y, projs[..., 3 * ds + 3 * dm:], gn_w, gn_b, H).to(dtype)
    assert_close(out[..., out_col:], ref, dtype, f"slot+gate out_col={out_col}")
    assert out[..., :out_col].abs().max().item() == 0.0


ATTEND_CASES = [
    # (dtype, B, L, dm, H, C)
    (torch.float32, 2, 192, 256, 4, 64),
    (torch.bfloat16, 2, 192, 256, 4, 64),
    (torch.bfloat16, 1, 256, 512, 8, 32),    # C < row tile
    (torch.float32, 1, 256, 256, 4, 128),    # C > row tile: carried within-chunk state
    (torch.bfloat16, 1, 256, 768, 8, 128),   # hd 96
    (torch.bfloat16, 1, 256, 1024, 8, 64),   # hd 128
    (torch.float32, 1, 128, 512, 4, 32),     # hd 128
    (torch.bfloat16, 1, 192, 384, 8, 48),    # hd 48, C 48: chunk-confined tiles
    (torch.float32, 1, 160, 320, 4, 80),     # hd 80, C 80 > TC, not a multiple of it
    (torch.bfloat16, 1, 192, 256, 16, 96),   # hd 16, C 96
]


@pytest.mark.parametrize("dtype,B,L,dm,H,C", ATTEND_CASES)
@pytest.mark.parametrize("phi,reverse", [(True, False), (False, False), (False, True)])
def test_slot_attend(dev, dtype, B, L, dm, H, C, phi, reverse):
    """The slot recurrence without GroupNorm/gate on three column blocks of one buffer in a
    shuffled order (v, q, k, plus an unused block), forwards or backwards in time; then with
    the feature map's chain rule applied as the outputs are stored."""
    _say("slot_attend", dtype, B, L, dm, H, C, phi, reverse)
    g = torch.Generator().manual_seed(L + dm + C + phi + 2 * reverse)
    hd = dm // H
    base = (0.5 * torch.randn(B, L, 4 * dm, generator=g)).to(dtype)
    q_col, k_col, v_col = dm, 2 * dm, 0
    gamma = (0.9 + 0.099 * torch.rand(H, generator=g)).to(dtype)
    q = base[..., q_col:q_col + dm].float().view(B, L, H, hd)
    k = base[..., k_col:k_col + dm].float().view(B, L, H, hd)
    v = base[..., v_col:v_col + dm].float().view(B, L, H, hd)
    if phi:
        q, k = oracle.phi(q), oracle.phi(k)
    if reverse:
        q, k, v = q.flip(1), k.flip(1), v.flip(1)
    ref, _ = oracle.attend_chunked(q, k, v, gamma, C, dtype)
    if reverse:
        ref = ref.flip(1)
    out = torch.zeros(B, L, 8 + dm, device=dev, dtype=dtype)
    _ops.slot_attend(base.to(dev), q_col, k_col, v_col, gamma.to(dev), dm, H, C, phi, out, 8, reverse=reverse)
    assert out[..., :8].abs().max().item() == 0.0
    got = out[..., 8:].float().cpu()
    lim = 1e-4 if dtype == torch.float32 else 2e-2
    err = ((got - ref.reshape(B, L, dm)).abs().max() / ref.abs().max()).item()
    assert err <= lim, err
    # chain: out *= phi'(z), z from a buffer with out's column layout (d phi -> d q / d k)
    z = torch.randn(B, L, 8 + dm, generator=g).to(dtype)
    zz = z[..., 8:].float()
    ref_c = ref.reshape(B, L, dm) * torch.where(zz > 0, torch.ones_like(zz), torch.exp(zz))
    out.zero_()
    _ops.slot_attend(base.to(dev), q_col, k_col, v_col, gamma.to(dev), dm, H, C, phi, out, 8, reverse=reverse,
                     chain=z.to(dev))
    got = out[..., 8:].float().cpu()
    err = ((got - ref_c).abs().max() / ref_c.abs().max()).item()
    assert err <= lim, ("chain", err)


@pytest.mark.parametrize("C,L", [(64, 1024), (48, 960), (96, 960), (80, 960)])
def test_slot_segments_option(dev, C, L):
    """Different segment lengths (state pre-pass on/off) give the same result, and the
    oracle's; for chunks that do not divide the row tile the segments hold whole chunks."""
    dm, ds, H, B = 256, 64, 4, 1
    _say("slot segments", C, L)
    projs, gamma, gn_w, gn_b = slot_inputs(B, L, dm, ds, H, torch.float32, seed=3 + C)
    outs = []
    for st in (1, 2, 3, 16):
        with _ops.option("slot_seg_tiles", st):
            outs.append(_run_slot(dev, projs, gamma, gn_w, gn_b, dm, ds, H, C)[0])
    for o in outs[1:]:
        assert_close(o, outs[0], torch.float32, "segment invariance")
    y, _ = oracle.slot_chunked(projs, gamma, dm, ds, H, C, torch.float32)
    ref = oracle.gnorm_gate(y, projs[..., 3 * ds + 3 * dm:], gn_w, gn_b, H)
    assert_close(outs[0][..., ds:], ref, torch.float32, "slot+gate")


@pytest.mark.parametrize("dm,H", [(200, 5), (576, 4)])  # hd 40 (not a multiple of 16), hd 144
def test_slot_unsupported_head_dim(dev, dm, H):
    projs, gamma, gn_w, gn_b = slot_inputs(1, 64, dm, 64, H, torch.bfloat16)
    with pytest.raises(_ops.HdcmError):
        _run_slot(dev, projs, gamma, gn_w, gn_b, dm, 64, H, 64)


# ----------------------------------------------------------------------------- skinny decode GEMM
@pytest.mark.parametrize("M,N,K,bias,res", [
    (16, 8576, 2048, True, False),    # d_model 2048 in_proj of a B=16 decode step
    (16, 2048, 2176, False, True),    # its out_proj with the residual add
    (16, 50304, 2048, False, False),  # the tied LM head
    (7, 3264, 768, True, False),
    (16, 768, 832, False, True),
    (1, 100, 64, True, True),
    (5, 33, 3072, False, False),
    # N >= 2048 runs the LDS-staged kernel: fewer K steps than waves, ragged N, K = 3072
    (3, 2048, 64, True, True),
    (9, 2050, 1024, False, True),
    (16, 4096, 3072, True, False),
    # more than 384 tiles with K <= 2048: two tiles per workgroup (odd tile count: the last
    # workgroup's second tile lies past N)
    (16, 8576, 2048, True, False), (5, 6210, 512, False, True),
])
def test_skinny_gemm(dev, M, N, K, bias, res):
    """bf16 operands, fp32 accumulation, one rounding: against torch fp32 on the same
    bf16 operands (max error a bf16 rounding of the result plus fp32 summation order)."""
    _say("skinny", M, N, K, bias, res)
    g = torch.Generator().manual_seed(M * 7 + N + K)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    b = (0.1 * torch.randn(N, generator=g)).to(torch.bfloat16) if bias else None
    r = torch.randn(M, N, generator=g).to(torch.bfloat16) if res else None
    ref = A.float() @ W.float().t()
    if bias:
        ref = ref + b.float()
    if res:
        ref = ref + r.float()
    out = _ops.skinny_linear(A.to(dev), W.to(dev), None if b is None else b.to(dev),
                             None if r is None else r.to(dev))
    torch.cuda.synchronize()
    err = (out.float().cpu() - ref).abs()
    assert (err <= 2 ** -8 * ref.abs() + 1e-3).all(), f"max err {err.max().item()}"


@pytest.mark.parametrize("M,N,K,bias,res,ln", [
    (16, 2048, 2176, False, True, True),    # the d_model 2048 decode out_proj (LayerNorm folded)
    (16, 2048, 2176, False, True, False),
    (16, 8576, 2048, True, False, False),   # its in_proj
    (9, 2050, 1024, False, True, False),    # ragged last workgroup
    (9, 2056, 1024, False, True, True),     # 16-column tiles: the last one half full
    (3, 4100, 96, True, True, False),
])
def test_skinny_columns_per_workgroup(dev, M, N, K, bias, res, ln):
    """8 output columns per workgroup (the MFMA's other 8 columns repeat them) give the same
    bits as 16: each output column's dot product runs in the same order either way."""
    _say("skinny cols", M, N, K, bias, res, ln)
    g = torch.Generator().manual_seed(M + N + K)
    A = (1.5 * torch.randn(M, K, generator=g) + 0.5).to(torch.bfloat16).to(dev)
    W = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(dev)
    b = (0.1 * torch.randn(N, generator=g)).to(torch.bfloat16).to(dev) if bias else None
    r = torch.randn(M, N, generator=g).to(torch.bfloat16).to(dev) if res else None
    outs = []
    for cols8_max_n in (0, 1 << 30):
        with _ops.option("skinny_cols8_max_n", cols8_max_n):
            outs.append(_ops.rowln_gemm(A, W, r) if ln else _ops.skinny_linear(A, W, b, r))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    ref = torch.nn.functional.layer_norm(A.float().cpu(), (K,), eps=1e-5) if ln else A.float().cpu()
    ref = ref @ W.float().cpu().t()
    if bias:
        ref = ref + b.float().cpu()
    if res:
        ref = ref + r.float().cpu()
    err = (outs[1].float().cpu() - ref).abs()
    assert (err <= 2 ** -8 * ref.abs() + 2e-3).all(), f"max err {err.max().item()}"


@pytest.mark.parametrize("M,N,K,bias,res,cols8", [
    (16, 8576, 2048, True, False, False),   # the d_model 2048 decode in_proj: 536 column tiles
    (16, 8208, 2048, False, True, False),   # one tile past a round of 512 workgroups
    (5, 16384, 1024, True, True, False),    # exactly two rounds' worth
    (16, 8576, 2048, True, False, True),    # 8-column tiles
    (16, 8584, 2048, True, False, False),   # the last tile half full
])
def test_skinny_fold_tail(dev, M, N, K, bias, res, cols8):
    """The tiles past one round of resident workgroups, taken as second tiles by the first
    workgroups, give the same bits as a second round of workgroups."""
    _say("skinny fold tail", M, N, K, bias, res, cols8)
    g = torch.Generator().manual_seed(N + K)
    A = (1.5 * torch.randn(M, K, generator=g) + 0.5).to(torch.bfloat16).to(dev)
    W = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(dev)
    b = (0.1 * torch.randn(N, generator=g)).to(torch.bfloat16).to(dev) if bias else None
    r = torch.randn(M, N, generator=g).to(torch.bfloat16).to(dev) if res else None
    outs = []
    with _ops.option("skinny_cols8_max_n", (1 << 30) if cols8 else 0):
        for fold in (0, 1):
            with _ops.option("skinny_fold_tail", fold):
                outs.append(_ops.skinny_linear(A, W, b, r))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    ref = A.float().cpu() @ W.float().cpu().t()
    if bias:
        ref = ref + b.float().cpu()
    if res:
        ref = ref + r.float().cpu()
    err = (outs[1].float().cpu() - ref).abs()
    assert (err <= 2 ** -8 * ref.abs() + 2e-3).all(), f"max err {err.max().item()}"


def _front_inputs(B, D, N, bias, seed):
    g = torch.Generator().manual_seed(seed)
    bf = torch.bfloat16
    p = dict(ln_w=(1 + 0.1 * torch.randn(D, generator=g)).to(bf), ln_b=(0.1 * torch.randn(D, generator=g)).to(bf),
             conv_w=(0.3 * torch.randn(D, 4, generator=g)).to(bf), conv_b=(0.1 * torch.randn(D, generator=g)).to(bf),
             W=(torch.randn(N, D, generator=g) / D ** 0.5).to(bf),
             b=(0.1 * torch.randn(N, generator=g)).to(bf) if bias else None,
             hist=(2 * torch.randn(B, 3, D, generator=g) + 0.3).to(bf))
    xs = [(2 * torch.randn(B, D, generator=g) - 0.4).to(bf) for _ in range(3)]
    return p, xs


@pytest.mark.parametrize("B,D,N,bias", [
    (16, 2048, 8576, True),   # the d_model 2048 in_proj: 536 tiles, second tiles on the first workgroups
    (5, 1024, 4480, True),    # d_model 1024: one round of workgroups
    (1, 768, 3456, False),    # one row, no bias
    (16, 512, 40000, True),   # more tiles than twice the resident workgroups: several rounds
    (3, 2048, 2056, True),    # the last tile half full
    (2, 32, 20, True),        # one K step (seven of eight waves idle), two tiles, the last one 4 wide
    (16, 64, 2048, False),    # two K steps, exactly one round
])
def test_norm_conv_in_proj_step(dev, B, D, N, bias):
    """The one-launch decode front against its two kernels (norm_conv_step, then skinny_linear
    over its output): the same bits for the conv rows, the projections and the shifted history,
    over three calls in a row (a new call tag each), with no wait timing out."""
    _say("norm_conv_in_proj_step", B, D, N, bias)
    p, xs = _front_inputs(B, D, N, bias, B * 7 + D + N)
    p = {k: (v.to(dev) if v is not None else None) for k, v in p.items()}
    h1, h2 = p["hist"].clone(), p["hist"].clone()
    for x in xs:
        x = x.to(dev)
        u1 = _ops.norm_conv_step(x, p["ln_w"], p["ln_b"], p["conv_w"], p["conv_b"], 1e-5, h1)
        o1 = _ops.skinny_linear(u1, p["W"], p["b"])
        u2, o2 = _ops.norm_conv_in_proj_step(x, p["ln_w"], p["ln_b"], p["conv_w"], p["conv_b"], 1e-5, h2, p["W"],
                                             p["b"])
        torch.cuda.synchronize()
        assert torch.equal(u1, u2)
        assert torch.equal(o1, o2)
        assert torch.equal(h1, h2)
    assert _ops.step_timeouts(dev) == 0
    # and against the plain-torch restatement of the projection
    ref = u2.float().cpu() @ p["W"].float().cpu().t() + (p["b"].float().cpu() if bias else 0)
    err = (o2.float().cpu() - ref).abs()
    assert (err <= 2 ** -8 * ref.abs() + 2e-3).all(), f"max err {err.max().item()}"


def test_norm_conv_in_proj_step_graph(dev):
    """The fused front recorded in a HIP graph: every replay (with eager calls of it between the
    replays, each advancing the call tag) matches the two-kernel path on the same inputs."""
    _say("norm_conv_in_proj_step graph")
    B, D, N = 16, 2048, 8576
    p, xs = _front_inputs(B, D, N, True, 99)
    p = {k: v.to(dev) for k, v in p.items()}
    x = xs[0].to(dev)
    hist = p["hist"].clone()
    u = torch.empty(B, D, device=dev, dtype=torch.bfloat16)
    o = torch.empty(B, N, device=dev, dtype=torch.bfloat16)
    args = (p["ln_w"], p["ln_b"], p["conv_w"], p["conv_b"], 1e-5)
    _ops.norm_conv_in_proj_step(x, *args, hist, p["W"], p["b"], u=u, out=o)  # the workspace exists before capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _ops.norm_conv_in_proj_step(x, *args, hist, p["W"], p["b"], u=u, out=o)
    g = torch.Generator().manual_seed(5)
    h_ref = hist.clone()
    scratch_hist = hist.clone()
    for rep in range(4):
        x.copy_((2 * torch.randn(B, D, generator=g)).to(torch.bfloat16))
        u_ref = _ops.norm_conv_step(x, *args, h_ref)
        o_ref = _ops.skinny_linear(u_ref, p["W"], p["b"])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(u, u_ref), rep
        assert torch.equal(o, o_ref), rep
        assert torch.equal(hist, h_ref), rep
        _ops.norm_conv_in_proj_step(x, *args, scratch_hist, p["W"], p["b"])  # an eager call between replays
        torch.cuda.synchronize()
    assert _ops.step_timeouts(dev) == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("hd,H,two", [(256, 4, True), (160, 3, True), (96, 2, False)])
def test_gnorm_gate_pass(dev, dtype, hd, H, two):
    """The GroupNorm + gate pass of wide heads against oracle.gnorm_gate on y1 + y2' (y2 with
    each head's halves exchanged), with its row statistics against the stored values."""
    _say("gnorm gate pass", dtype, hd, H, two)
    g = torch.Generator().manual_seed(hd + H)
    rows, dm = 300, hd * H
    y1 = (torch.randn(rows, dm, generator=g) + 0.3).to(dtype)
    y2 = torch.randn(rows, dm, generator=g).to(dtype) if two else None
    gate = torch.randn(rows, 2 * dm, generator=g).to(dtype)[:, dm // 2:dm // 2 + dm]  # a strided view
    gn_w = (1 + 0.2 * torch.randn(dm, generator=g)).to(dtype)
    gn_b = (0.1 * torch.randn(dm, generator=g)).to(dtype)
    y = y1.float()
    if two:
        y = y + y2.float().view(rows, H, 2, hd // 2).flip(2).reshape(rows, dm)
    ref = oracle.gnorm_gate(y.view(1, rows, H, hd), gate.float().view(1, rows, dm), gn_w, gn_b, H).view(rows, dm)
    out = torch.zeros(rows, dm + 8, dtype=dtype, device=dev)[:, 8:]
    stats = torch.zeros(H + 1, rows, 2, dtype=torch.float32, device=dev)
    _ops.gnorm_gate(y1.to(dev), y2.to(dev) if two else None, gate.to(dev), gn_w.to(dev), gn_b.to(dev), 1e-5, H,
                    out, row_stats=stats, stats_part=1)
    torch.cuda.synchronize()
    assert_close(out.cpu(), ref, dtype, "gnorm gate")
    o = out.float().cpu().view(rows, H, hd)
    torch.testing.assert_close(stats[1:].cpu(), torch.stack([o.sum(-1), (o * o).sum(-1)], -1).transpose(0, 1),
                               rtol=1e-5, atol=1e-4)
    assert (stats[0] == 0).all()


def test_skinny_gemm_in_place_residual(dev):
    """out may be the residual buffer itself."""
    g = torch.Generator().manual_seed(3)
    A = torch.randn(16, 512, generator=g).to(torch.bfloat16).to(dev)
    W = (torch.randn(256, 512, generator=g) / 512 ** 0.5).to(torch.bfloat16).to(dev)
    r = torch.randn(16, 256, generator=g).to(torch.bfloat16).to(dev)
    ref = (A.float() @ W.float().t() + r.float()).cpu()
    out = _ops.skinny_linear(A, W, residual=r, out=r)
    torch.cuda.synchronize()
    assert out.data_ptr() == r.data_ptr()
    err = (r.float().cpu() - ref).abs()
    assert (err <= 2 ** -8 * ref.abs() + 1e-3).all()


# ----------------------------------------------------------------------------- tiled GEMM
@pytest.mark.parametrize("M,N,K,bias", [
    (300, 100, 72, True), (100, 64, 40, False), (1000, 4480, 1024, True), (257, 260, 1152, False),
    (513, 4480, 1000, True), (700, 512, 160, True), (1, 8, 8, True), (256, 256, 64, False),
    (6000, 4480, 1024, True), (8400, 2500, 960, False), (8400, 2500, 960, True),
])
def test_tiled_gemm(dev, M, N, K, bias):
    """hdcm_gemm_fwd against torch fp32 on the same bf16 operands: partial tiles in every
    dimension (M, N not multiples of 256, K not a multiple of 64) and the bias epilogue; the
    last three shapes launch more workgroups than the GPU has CUs, one of them with an odd
    number of K steps."""
    _say("gemm", M, N, K, bias)
    g = torch.Generator().manual_seed(M + 3 * N + 7 * K)
    X = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    b = (0.1 * torch.randn(N, generator=g)).to(torch.bfloat16) if bias else None
    ref = X.float() @ W.float().t() + (b.float() if bias else 0.0)
    out = _ops.gemm(X.to(dev), W.to(dev), None if b is None else b.to(dev))
    torch.cuda.synchronize()
    err = (out.float().cpu() - ref).abs()
    assert (err <= 2 ** -8 * ref.abs() + 1e-3).all(), f"max err {err.max().item()}"


@pytest.mark.parametrize("M,N,K,mean", [
    (300, 100, 72, 0.3), (257, 260, 1152, 4.0), (4096, 1024, 1152, 0.0), (513, 768, 832, 2.0), (1, 8, 8, 1.0),
    # at most 16 rows and K a multiple of 32: the decode-step (skinny) kernels, narrow and wide
    (16, 1024, 1152, 3.0), (7, 768, 832, 0.5), (16, 2048, 2176, 1.0), (1, 2052, 64, 2.0), (3, 100, 3072, 0.0),
])
def test_rowln_gemm(dev, M, N, K, mean):
    """hdcm_rowln_gemm_fwd = res + LayerNorm(c) W^T (no affine, eps 1e-5) against torch fp32
    (F.layer_norm on the bf16 rows): rows with a large mean, ragged tiles, the few-row
    decode shapes; then in place."""
    _say("rowln_gemm", M, N, K, mean)
    g = torch.Generator().manual_seed(M + N + K)
    c = (1.5 * torch.randn(M, K, generator=g) + mean).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    r = torch.randn(M, N, generator=g).to(torch.bfloat16)
    ref = r.float() + torch.nn.functional.layer_norm(c.float(), (K,), eps=1e-5) @ W.float().t()
    cd, Wd, rd = c.to(dev), W.to(dev), r.to(dev)
    out = _ops.rowln_gemm(cd, Wd, rd)
    torch.cuda.synchronize()
    err = (out.float().cpu() - ref).abs()
    assert (err <= 2 ** -8 * ref.abs() + 2e-3).all(), f"max err {err.max().item()}"
    _ops.rowln_gemm(cd, Wd, rd, out=rd)  # out aliasing the residual
    torch.cuda.synchronize()
    assert torch.equal(rd.cpu(), out.cpu())


def _block_sums(vals, width):
    """[rows, cols] -> [rows, ceil(cols / width), 2] fp64 (sum, sum of squares) per column block."""
    v = vals.double()
    nb = -(-v.shape[1] // width)
    out = torch.zeros(v.shape[0], nb, 2, dtype=torch.float64)
    for i in range(nb):
        blk = v[:, i * width:(i + 1) * width]
        out[:, i, 0] = blk.sum(1)
        out[:, i, 1] = (blk * blk).sum(1)
    return out


def _check_stats(got, ref, what):
    torch.cuda.synchronize()
    g = got.double().cpu()
    tol = 1e-5 * ref.abs() + 1e-4
    bad = (g - ref).abs() > tol
    assert not bad.any(), f"{what}: {bad.sum().item()} sums off, max err {(g - ref).abs().max().item()}"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("ds,B,L", [(128, 2, 700), (80, 1, 3000), (64, 1, 32768)])
def test_ssm_row_stats(dev, dtype, ds, B, L):
    """The scan's per-row (sum, sum of squares) of its stored values over each 32-channel block
    (the last one partial for ds=80), written at the given pair column of a wider buffer whose
    other columns stay untouched; y unchanged by the option."""
    _say("ssm row stats", dtype, ds, B, L)
    projs, A_log = ssm_inputs(B, L, ds, dtype)
    pd, ad = projs.to(dev), A_log.to(dev)
    nb = _ops.ssm_stats_parts(ds)
    st = torch.full((nb + 2, B * L, 2), 7.0, device=dev)
    y = torch.empty(B, L, ds, device=dev, dtype=dtype)
    y0 = torch.empty_like(y)
    _ops.ssm(pd, ad, ds, y0)
    _ops.ssm(pd, ad, ds, y, row_stats=st, stats_part=1)
    torch.cuda.synchronize()
    assert torch.equal(y, y0)
    _check_stats(st[1:1 + nb].transpose(0, 1), _block_sums(y.cpu().reshape(B * L, ds), 32), "ssm row stats")
    assert (st[0] == 7).all() and (st[1 + nb:] == 7).all()


@pytest.mark.parametrize("dtype,B,L,dm,H,C,out_col", [
    (torch.bfloat16, 1, 512, 256, 4, 64, 64), (torch.float32, 2, 256, 256, 8, 64, 64),
    (torch.bfloat16, 1, 512, 512, 4, 128, 64), (torch.bfloat16, 2, 256, 256, 8, 64, 4),  # 8-byte store path
    (torch.float32, 1, 384, 384, 4, 64, 64)])
def test_slot_gate_row_stats(dev, dtype, B, L, dm, H, C, out_col):
    """slot_gate's per-row (sum, sum of squares) of its stored values, one pair per head."""
    _say("slot row stats", dtype, B, L, dm, H, C, out_col)
    ds = 64
    projs, gamma, gn_w, gn_b = slot_inputs(B, L, dm, ds, H, dtype, seed=L + dm)
    pd = projs.to(dev)
    out = torch.zeros(B, L, out_col + dm, device=dev, dtype=dtype)
    ws = _ops.slot_workspace(pd, dm, H, C)
    _ops.slot_state(pd, 3 * ds, gamma.to(dev), dm, H, C, ws)
    st = torch.full((H + 1, B * L, 2), 7.0, device=dev)
    _ops.slot_gate(pd, 3 * ds, gamma.to(dev), gn_w.to(dev), gn_b.to(dev), 1e-5, ws, out, out_col, dm, H, C,
                   row_stats=st, stats_part=1)
    vals = out[..., out_col:].cpu().reshape(B * L, dm)
    _check_stats(st[1:].transpose(0, 1), _block_sums(vals, dm // H), "slot row stats")
    assert (st[0] == 7).all()


@pytest.mark.parametrize("M,N,K,mean", [
    (300, 264, 1152, 0.3), (4096, 1024, 1152, 4.0), (513, 768, 832, 2.0), (17, 8, 64, 1.0), (1000, 2048, 2176, 0.0)])
def test_rowln_gemm_stats(dev, M, N, K, mean):
    """hdcm_rowln_gemm_stats_fwd with row statistics supplied as 64-column partial sums and the
    weight row sums from hdcm_row_sums_fwd: the bound of test_rowln_gemm against torch fp32,
    then in place."""
    _say("rowln_gemm_stats", M, N, K, mean)
    g = torch.Generator().manual_seed(M + N + K + 1)
    c = (1.5 * torch.randn(M, K, generator=g) + mean).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    r = torch.randn(M, N, generator=g).to(torch.bfloat16)
    ref = r.float() + torch.nn.functional.layer_norm(c.float(), (K,), eps=1e-5) @ W.float().t()
    cd, Wd, rd = c.to(dev), W.to(dev), r.to(dev)
    ws = _ops.row_sums(Wd)
    torch.cuda.synchronize()
    assert torch.allclose(ws.cpu().double(), W.double().sum(1), rtol=1e-5, atol=1e-4)
    st = _block_sums(c, 64).float().transpose(0, 1).contiguous().to(dev)
    out = _ops.rowln_gemm_stats(cd, Wd, ws, st, rd)
    torch.cuda.synchronize()
    err = (out.float().cpu() - ref).abs()
    assert (err <= 2 ** -8 * ref.abs() + 2e-3).all(), f"max err {err.max().item()}"
    _ops.rowln_gemm_stats(cd, Wd, ws, st, rd, out=rd)  # out aliasing the residual
    torch.cuda.synchronize()
    assert torch.equal(rd.cpu(), out.cpu())


def test_fused_out_proj_matches_unfused(dev):
    """A bf16 model forward with the LayerNorm folded into out_proj against the same model
    with the row LayerNorm kernel and addmm."""
    from hdcmamba_amd import HdcMamba9v3Model, set_fused_out_proj

    torch.manual_seed(0)
    m = HdcMamba9v3Model(256, 2, 64, 32, num_heads=4, chunk_size=64).to(torch.bfloat16).to(dev).eval()
    x = torch.randn(2, 200, 256, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        a = m(x)
        set_fused_out_proj(m, False)
        b = m(x)
    err = ((a.float() - b.float()).norm() / b.float().norm()).item()
    _say(f"  fused vs unfused normwise {err:.2e}")
    assert err < 1e-2


# ----------------------------------------------------------------------------- norm_conv backward
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,L,D", [(2, 1, 256), (2, 5, 256), (1, 300, 1024), (2, 700, 768), (1, 64, 2048),
                                   (3, 131, 512), (1, 70, 1280), (2, 40, 1536),
                                   (2, 37, 3072), (1, 20, 2560)])  # rows shared by a workgroup's waves
def test_norm_conv_backward(dev, dtype, B, L, D):
    """FusedNormConv1dFunction's backward against autograd through the oracle (fp64 for fp32
    inputs): dx elementwise, the parameter gradients (sums over B*L rows) normwise.  D above
    2048 takes the kernel whose four waves share each row."""
    from hdcmamba_amd import FusedNormConv1dFunction

    _say("norm_conv bwd", dtype, B, L, D)
    g = torch.Generator().manual_seed(B * 1000 + L + D)
    x = (2 * torch.randn(B, L, D, generator=g) + 0.5).to(dtype)
    w = (1 + 0.2 * torch.randn(D, generator=g)).to(dtype)
    b = (0.3 * torch.randn(D, generator=g)).to(dtype)
    cw = (0.5 * torch.randn(D, 4, generator=g)).to(dtype)
    cb = (0.1 * torch.randn(D, generator=g)).to(dtype)
    go = torch.randn(B, L, D, generator=g).to(dtype)
    ref_dt = torch.float64 if dtype == torch.float32 else torch.float32
    ins = [t.to(ref_dt).requires_grad_() for t in (x, w, b, cw, cb)]
    fn = lambda *a: oracle.norm_conv(*[t.float() for t in a], 1e-5).to(ref_dt)
    if ref_dt == torch.float64:  # the oracle computes in fp32; redo its math in fp64 for the reference
        def fn(xx, ww, bb, cww, cbb):
            mean = xx.mean(-1, keepdim=True)
            xc = xx - mean
            u = xc * torch.rsqrt((xc * xc).mean(-1, keepdim=True) + 1e-5) * ww + bb
            up = torch.cat([bb.expand(xx.shape[0], 3, D), u], 1)
            return sum(up[:, k:k + L] * cww[:, k] for k in range(4)) + cbb
        torch.testing.assert_close(fn(*[t.detach() for t in ins]).float(),
                                   oracle.norm_conv(x, w, b, cw, cb, 1e-5).float(), atol=2e-5, rtol=2e-5)
    refs = torch.autograd.grad(fn(*ins), ins, go.to(ref_dt))
    xd = x.to(dev).requires_grad_()
    params = [t.to(dev).requires_grad_() for t in (w, b, cw, cb)]
    y = FusedNormConv1dFunction.apply(xd, *params, 1e-5)
    y.backward(go.to(dev))
    got = [xd.grad] + [p.grad for p in params]
    names = ["dx", "d_ln_w", "d_ln_b", "d_conv_w", "d_conv_b"]
    for gt, rf, name in zip(got, refs, names):
        assert gt.dtype == dtype and gt.shape == rf.shape, name
        if name == "dx":
            assert_close(gt, rf.to(torch.float32), dtype, name)
        else:
            err = ((gt.float().cpu() - rf.float()).norm() / rf.float().norm()).item()
            _say("  ", name, "normwise", err)
            assert err <= (1e-4 if dtype == torch.float32 else 2e-2), f"{name}: {err}"
