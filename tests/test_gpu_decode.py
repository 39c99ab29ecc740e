"""Prefill -> recurrent decode on the GPU.

The decode semantics are the chunked forward continued token by token: the chunk grid is
the prefill's (its left padding to a multiple of C), so a prefill of n rows followed by k
steps equals oracle.block_forward_stream(x[:, :n+k], n_prefill=n).  Tolerances: fp32
1e-4 elementwise, bf16 2e-2 (normwise for multi-layer outputs).
"""
import pytest
import torch

import oracle
from cfgs import (WORKLOADS, assert_close, assert_close_normwise, lm_input, make_lm, max_rel, oracle_cfg,
                  reinit_block_)

pytestmark = pytest.mark.gpu


def _sd(m):
    return {k: v.detach().cpu() for k, v in m.state_dict().items()}


def _say(*a):
    print(*a, flush=True)


def _block(dm, ds, H, C, dtype, seed):
    from hdcmamba_amd import HdcMamba9v3Block

    torch.manual_seed(seed)
    return reinit_block_(HdcMamba9v3Block(dm, ds, H, C), seed=seed, decays_uniform=True).eval().to(dtype)


BLOCK_CASES = [
    # (dtype, B, dm, ds, H, C, n_prefill, n_decode)
    (torch.float32, 2, 256, 64, 8, 16, 40, 30),    # hd 32, prefill padded by 8, 2 chunk ends
    (torch.float32, 1, 512, 64, 8, 32, 64, 40),    # hd 64, aligned prefill
    (torch.bfloat16, 2, 512, 128, 8, 64, 130, 70),  # hd 64, prefill padded by 62
    (torch.bfloat16, 1, 768, 64, 8, 64, 64, 66),   # hd 96
    (torch.bfloat16, 2, 768, 64, 16, 48, 100, 60),  # hd 48, C 48 (chunk-confined tiles), padded prefill
    (torch.float32, 1, 320, 64, 4, 80, 160, 90),   # hd 80, C 80 > TC (fp32 tile 32)
    (torch.bfloat16, 1, 256, 64, 16, 96, 96, 100),  # hd 16, C 96: tiles of 64 + 32 rows
]


@pytest.mark.parametrize("dtype,B,dm,ds,H,C,n_pre,n_dec", BLOCK_CASES)
def test_block_prefill_then_steps(dev, dtype, B, dm, ds, H, C, n_pre, n_dec):
    _say("block decode", dtype, B, dm, ds, H, C, n_pre, n_dec)
    blk = _block(dm, ds, H, C, dtype, seed=n_pre + dm)
    x = torch.randn(B, n_pre + n_dec, dm, generator=torch.Generator().manual_seed(dm)).to(dtype)
    ref = oracle.block_forward_stream(_sd(blk), x, oracle_cfg(blk), n_pre)
    blk = blk.to(dev)
    xd = x.to(dev)
    with torch.no_grad():
        y0, st = blk.prefill(xd[:, :n_pre])
        ys = [blk.step(xd[:, n_pre + t].contiguous(), st) for t in range(n_dec)]
    assert_close(y0, ref[:, :n_pre], dtype, "prefill rows")
    got = torch.stack(ys, 1)
    _say("  decode max rel", max_rel(got, ref[:, n_pre:]))
    assert_close(got, ref[:, n_pre:], dtype, "decode rows")
    assert st.pos == (n_pre + (C - n_pre % C) % C + n_dec) % C


@pytest.mark.parametrize("dtype,B,dm,ds,H,C,n_pre,n_dec", [
    (torch.float32, 2, 256, 64, 8, 16, 40, 30), (torch.bfloat16, 2, 512, 128, 8, 64, 130, 70),
    (torch.bfloat16, 16, 2048, 128, 32, 64, 128, 66)])  # C5 width (fused decode front)
def test_block_steps_and_states_match_oracle_step(dev, dtype, B, dm, ds, H, C, n_pre, n_dec):
    """The GPU prefill's carried state and every decode step against the oracle's recurrent
    step (oracle.block_prefill_state / block_step), which uses the step's own rounding points:
    outputs per token and, after the last step, the conv history, the SSM state and both slot
    states (S_intra compared where it is live, i.e. off a chunk boundary)."""
    _say("block steps vs oracle step", dtype, B, dm, ds, H, C, n_pre, n_dec)
    blk = _block(dm, ds, H, C, dtype, seed=n_pre + dm + 1)
    x = torch.randn(B, n_pre + n_dec, dm, generator=torch.Generator().manual_seed(dm + 7)).to(dtype)
    cfg = oracle_cfg(blk)
    sd = _sd(blk)
    y0_ref, ost = oracle.block_prefill_state(sd, x[:, :n_pre], cfg)
    refs = [oracle.block_step(sd, x[:, n_pre + t], ost, cfg) for t in range(n_dec)]
    blk = blk.to(dev)
    xd = x.to(dev)
    with torch.no_grad():
        y0, st = blk.prefill(xd[:, :n_pre])
        assert_close(st.conv, x[:, n_pre - 3:n_pre], dtype, "prefill conv history")
        ys = [blk.step(xd[:, n_pre + t].contiguous(), st) for t in range(n_dec)]
    assert_close(y0, y0_ref, dtype, "prefill rows")
    assert_close(torch.stack(ys, 1), torch.stack(refs, 1), dtype, "decode rows")
    assert st.pos == ost["pos"]
    assert torch.equal(st.conv.cpu(), ost["conv"])
    assert_close_normwise(st.h, ost["h"], dtype, "SSM state")
    assert_close_normwise(st.S_prev, ost["S_prev"], dtype, "slot state at the chunk boundary")
    if ost["pos"] != 0:
        assert_close_normwise(st.S_intra, ost["S_intra"], dtype, "slot state inside the chunk")


@pytest.mark.parametrize("B,n_pre,n_dec", [(2, 8192, 32), (16, 8192, 8)])
def test_block_c5_width_prefill_then_steps(dev, B, n_pre, n_dec):
    """A block of the 48-layer d_model 2048 decode workload (32 heads, d_state 128, chunk 64)
    against the oracle: an 8192-row prefill, then single-token steps.  At B=2 the slot kernels
    cut each sequence into segments and the prefill's out_proj is the GEMM with the folded
    LayerNorm; at B=16 (B*H = 512 workgroups) every (sequence, head) is one segment walked
    from row 0 with no state pre-pass, and the prefill takes the LayerNorm kernel and the
    library out_proj."""
    from hdcmamba_amd import _ops

    dm, ds, H, C = 2048, 128, 32, 64
    dtype = torch.bfloat16
    _say("c5-width block decode", B, n_pre, n_dec)
    lib = _ops.lib()
    nseg = lib.hdcm_slot_workspace_bytes(B, n_pre, dm, H, C, _ops.HDCM_BF16) // (2 * B * H * 64 * 64 * 4)
    assert (nseg == 1) == (B == 16), nseg
    blk = _block(dm, ds, H, C, dtype, seed=2048 + B)
    x = torch.randn(B, n_pre + n_dec, dm, generator=torch.Generator().manual_seed(B)).to(dtype)
    ref = oracle.block_forward_stream(_sd(blk), x, oracle_cfg(blk), n_pre)
    blk = blk.to(dev)
    xd = x.to(dev)
    with torch.no_grad():
        y0, st = blk.prefill(xd[:, :n_pre])
        ys = [blk.step(xd[:, n_pre + t].contiguous(), st) for t in range(n_dec)]
    _say("  prefill max rel", max_rel(y0, ref[:, :n_pre]))
    assert_close(y0, ref[:, :n_pre], dtype, "prefill rows")
    got = torch.stack(ys, 1)
    _say("  decode max rel", max_rel(got, ref[:, n_pre:]))
    assert_close(got, ref[:, n_pre:], dtype, "decode rows")


def test_steps_from_empty_state_equal_forward(dev):
    """Token-by-token from the empty state reproduces the chunked forward of an aligned
    sequence (both start their chunk grid at row 0)."""
    dm, ds, H, C, B, L = 256, 64, 4, 16, 2, 48
    blk = _block(dm, ds, H, C, torch.float32, seed=2).to(dev)
    x = torch.randn(B, L, dm, generator=torch.Generator().manual_seed(3)).to(dev)
    with torch.no_grad():
        y, _ = blk(x)
        st = blk.new_state(B, dev, torch.float32)
        ys = torch.stack([blk.step(x[:, t].contiguous(), st) for t in range(L)], 1)
    assert_close(ys, y, torch.float32, "steps vs forward")


def test_model_prefill_then_steps(dev):
    from hdcmamba_amd import HdcMamba9v3Model

    dm, ds, H, C, B, n_pre, n_dec = 256, 64, 4, 32, 2, 50, 20
    _say("model decode")
    torch.manual_seed(4)
    m = HdcMamba9v3Model(dm, 3, ds, 32, num_heads=H, chunk_size=C)
    for i, blk in enumerate(m.layers):
        reinit_block_(blk, seed=20 + i, decays_uniform=True)
    m = m.eval()
    x = torch.randn(B, n_pre + n_dec, dm, generator=torch.Generator().manual_seed(5))
    ref = oracle.model_forward(_sd(m), x, oracle.BlockCfg(dm, ds, H, C), 3, n_prefill=n_pre)
    m = m.to(dev)
    xd = x.to(dev)
    y0, states = m.prefill(xd[:, :n_pre])
    ys = torch.stack([m.step(xd[:, n_pre + t].contiguous(), states) for t in range(n_dec)], 1)
    assert_close(y0, ref[:, :n_pre], torch.float32, "model prefill")
    assert_close(ys, ref[:, n_pre:], torch.float32, "model decode")


def test_lm_prefill_then_steps_small(dev):
    """2-layer d_model 768 LM in bf16: prefill logits of the last position, then decode
    logits, against the oracle (normwise)."""
    _say("lm decode small")
    lm = make_lm("lm_c3", n_layers=2).to(torch.bfloat16)
    B, n_pre, n_dec = 2, 200, 12
    ids = lm_input("lm_c3", B=B, L=n_pre + n_dec)
    ref = oracle.lm_forward(_sd(lm), ids, oracle.BlockCfg(768, 64, 12, 64), 2, n_prefill=n_pre)
    lm = lm.to(dev)
    idd = ids.to(dev)
    last, states = lm.prefill(idd[:, :n_pre])
    steps = torch.stack([lm.step(idd[:, n_pre + t].contiguous(), states) for t in range(n_dec)], 1)
    assert_close_normwise(last[:, -1], ref[:, n_pre - 1], torch.bfloat16, "prefill last logits")
    assert_close_normwise(steps, ref[:, n_pre:], torch.bfloat16, "decode logits")


def test_lm_c5_prefill_decode_matches_forward(dev):
    """48-layer d_model 2048 LM, B=16: prefill 8192 tokens, 256 decode steps; the decode
    logits equal the chunked forward over all 8448 tokens (8448 = 132 chunks, so both runs
    share the chunk grid).  bf16 normwise 2e-2 per step's logits."""
    cfg = WORKLOADS["lm_c5"]
    B, L, K = cfg["B"], cfg["L"], cfg["decode_steps"]
    _say("lm_c5 build")
    lm = make_lm("lm_c5").to(torch.bfloat16).to(dev)
    ids = lm_input("lm_c5", B=B, L=L + K).to(dev)
    with torch.no_grad():
        _say("lm_c5 full forward", B, L + K)
        y = lm.backbone(lm.embedding(ids))
        ref = lm._logits(y[:, L - 1:])  # positions L-1 .. L+K-1
        del y
        _say("lm_c5 prefill", B, L)
        last, states = lm.prefill(ids[:, :L])
        assert_close_normwise(last[:, -1], ref[:, 0], torch.bfloat16, "prefill last logits")
        _say("lm_c5 decode", K)
        worst = 0.0
        for t in range(K):
            logits = lm.step(ids[:, L + t].contiguous(), states)
            worst = max(worst, max_rel(logits, ref[:, 1 + t]))
        _say("  worst step normwise", worst)
    assert worst <= 2e-2


def test_decode_graph_replays_match_eager(dev):
    """Every replay of the captured decode step equals an eager step on a copy of the same
    states; eager work and synchronisations run between the replays, and the replays cross
    a chunk boundary (device-side chunk offset)."""
    from hdcmamba_amd.lm import _clone_state

    _say("decode graph")
    lm = make_lm("lm_c3", n_layers=2).to(torch.bfloat16).to(dev)
    B, n_pre, n_dec = 4, 100, 40  # prefill pads to 128; 70 replays cross the chunk end at offset 63
    ids = lm_input("lm_c3", B=B, L=n_pre + n_dec + 30).to(dev)
    _, states = lm.prefill(ids[:, :n_pre])
    eager_states = [_clone_state(st) for st in states]
    g = lm.capture_decode(states)
    # the first replays run from offset 0; step through a whole chunk boundary too
    for t in range(n_dec + 30):
        tok = ids[:, n_pre + t].contiguous()
        want = lm.step(tok, eager_states)
        torch.cuda.synchronize()
        got = g.step(tok).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, want) or max_rel(got, want) < 1e-3, f"replay {t}: {max_rel(got, want)}"
    assert states[0].pos == eager_states[0].pos
    for a, b in zip(states, eager_states):
        torch.testing.assert_close(a.S_prev, b.S_prev, atol=1e-3, rtol=1e-3)
        torch.testing.assert_close(a.h, b.h, atol=1e-3, rtol=1e-3)
