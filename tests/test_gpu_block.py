"""Block / model / LM forward on the GPU against the CPU oracle (intended semantics)."""
import pytest
import torch

import oracle
from cfgs import (WORKLOADS, assert_close, assert_close_normwise, block_input, lm_input, make_block, make_lm, max_rel,
                  oracle_cfg)

pytestmark = pytest.mark.gpu


def _sd(m):
    return {k: v.detach().cpu() for k, v in m.state_dict().items()}


@pytest.mark.parametrize("name", ["block_c1", "block_c2"])
def test_block_workload(dev, name):
    print("block", name, flush=True)
    cfg = WORKLOADS[name]
    blk = make_block(name).to(cfg["dtype"])
    x = block_input(name)
    ref = oracle.block_forward(_sd(blk), x, oracle_cfg(blk))
    blk = blk.to(dev)
    with torch.no_grad():
        y, none = blk(x.to(dev))
    assert none is None
    assert y.shape == x.shape and y.dtype == x.dtype
    print("max rel", max_rel(y, ref), flush=True)
    assert_close(y, ref, cfg["dtype"], name)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("L,C", [(100, 64), (300, 128), (1, 256)])
def test_block_padding(dev, dtype, L, C):
    """Lengths that are not a multiple of the chunk are left-padded like the reference."""
    print("block pad", dtype, L, C, flush=True)
    from hdcmamba_amd import HdcMamba9v3Block
    from cfgs import reinit_block_

    torch.manual_seed(5)
    blk = reinit_block_(HdcMamba9v3Block(256, 64, 4, C), seed=5).eval().to(dtype)
    x = torch.randn(2, L, 256, generator=torch.Generator().manual_seed(L)).to(dtype)
    ref = oracle.block_forward(_sd(blk), x, oracle_cfg(blk))
    with torch.no_grad():
        y, _ = blk.to(dev)(x.to(dev))
    assert_close(y, ref, dtype, f"pad L={L} C={C}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_default_heads_hd128(dev, dtype):
    """d_model 1024 with the constructor's default num_heads=8 (head dim 128), the shape a
    plain HdcMamba9v3Model(1024, n, 128, slots) builds."""
    print("block hd128", dtype, flush=True)
    from hdcmamba_amd import HdcMamba9v3Block
    from cfgs import reinit_block_

    torch.manual_seed(11)
    blk = reinit_block_(HdcMamba9v3Block(1024, 128, chunk_size=64), seed=11).eval().to(dtype)
    assert blk.head_dim == 128
    x = torch.randn(1, 320, 1024, generator=torch.Generator().manual_seed(12)).to(dtype)
    ref = oracle.block_forward(_sd(blk), x, oracle_cfg(blk))
    with torch.no_grad():
        y, _ = blk.to(dev)(x.to(dev))
    print("max rel", max_rel(y, ref), flush=True)
    assert_close(y, ref, dtype, f"hd128 {dtype}")


@pytest.mark.parametrize("dtype,dm,H,C,L", [
    (torch.bfloat16, 768, 16, 48, 200),   # hd 48, C 48: one chunk per 64-row tile, left pad 40
    (torch.float32, 640, 8, 96, 300),     # hd 80, C 96: tiles of 32 rows, three per chunk
    (torch.bfloat16, 256, 16, 80, 170),   # hd 16, C 80: tiles of 64 + 16 rows per chunk
    (torch.bfloat16, 896, 8, 64, 130),    # hd 112
])
def test_block_general_head_dims_and_chunks(dev, dtype, dm, H, C, L):
    """Head dims that are multiples of 16 but not of 32 and chunk sizes that neither divide
    the row tile nor are multiples of it, through the whole block (padding, SSM, slot + gate,
    the out_proj fold in bf16)."""
    print("block general", dtype, dm, H, C, L, flush=True)
    from hdcmamba_amd import HdcMamba9v3Block
    from cfgs import reinit_block_

    torch.manual_seed(dm + C)
    blk = reinit_block_(HdcMamba9v3Block(dm, 64, H, C), seed=dm + C, decays_uniform=True).eval().to(dtype)
    x = torch.randn(2, L, dm, generator=torch.Generator().manual_seed(L)).to(dtype)
    ref = oracle.block_forward(_sd(blk), x, oracle_cfg(blk))
    with torch.no_grad():
        y, _ = blk.to(dev)(x.to(dev))
    print("max rel", max_rel(y, ref), flush=True)
    assert_close(y, ref, dtype, f"dm={dm} H={H} C={C}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dm,H,C,L", [(512, 2, 64, 200), (640, 4, 48, 150)])
def test_block_wide_heads(dev, dtype, dm, H, C, L):
    """Head dims above 128 (256, and 160 with chunk 48): each head as two sub-heads of the plain
    slot pass plus the crossed key/value-block terms, then the GroupNorm over the whole head,
    through the whole block (padding, the out_proj fold in bf16); prefill state hand-off and the
    differentiable mixer are not built for them and raise."""
    print("block wide heads", dtype, dm, H, C, L, flush=True)
    from hdcmamba_amd import HdcMamba9v3Block
    from cfgs import reinit_block_

    torch.manual_seed(dm + H)
    blk = reinit_block_(HdcMamba9v3Block(dm, 64, H, C), seed=dm + H, decays_uniform=True).eval().to(dtype)
    assert blk.head_dim > 128
    x = torch.randn(2, L, dm, generator=torch.Generator().manual_seed(L)).to(dtype)
    ref = oracle.block_forward(_sd(blk), x, oracle_cfg(blk))
    blk = blk.to(dev)
    with torch.no_grad():
        y, _ = blk(x.to(dev))
    print("max rel", max_rel(y, ref), flush=True)
    assert_close(y, ref, dtype, f"dm={dm} H={H} C={C}")
    with torch.no_grad(), pytest.raises(RuntimeError):
        blk.prefill(x.to(dev))


def test_model_and_lm_small(dev):
    """2-layer LM (d_model 768, heads 12) at B=2, L=512 through embedding, blocks, norms, tied head."""
    print("lm small", flush=True)
    lm = make_lm("lm_c3", n_layers=2).to(torch.bfloat16)
    ids = lm_input("lm_c3", B=2, L=512)
    sd = _sd(lm)
    from oracle import BlockCfg
    cfg = BlockCfg(768, 64, 12, 64)
    ref = oracle.lm_forward(sd, ids, cfg, 2)
    with torch.no_grad():
        logits = lm.to(dev)(ids.to(dev))
    print("max rel", max_rel(logits, ref), flush=True)
    assert_close_normwise(logits, ref, torch.bfloat16, "lm logits")


def test_cpu_tensor_raises():
    """The product path has no CPU fallback."""
    from hdcmamba_amd import HdcMamba9v3Block

    blk = HdcMamba9v3Block(64, 16, 2, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        blk(torch.randn(1, 64, 64))


@pytest.mark.parametrize("L", [192, 100])
def test_model_inplace_stream(dev, L):
    """HdcMamba9v3Model under no_grad updates one residual stream in place; with a length
    that needs padding the pad rows must be re-zeroed before every block."""
    print("model inplace", L, flush=True)
    from hdcmamba_amd import HdcMamba9v3Model
    from cfgs import reinit_block_

    torch.manual_seed(3)
    m = HdcMamba9v3Model(256, 3, 64, 32, num_heads=4, chunk_size=64)
    for i, blk in enumerate(m.layers):
        reinit_block_(blk, seed=10 + i)
    m = m.eval()
    x = torch.randn(2, L, 256, generator=torch.Generator().manual_seed(L))
    ref = oracle.model_forward(_sd(m), x, oracle.BlockCfg(256, 64, 4, 64), 3)
    with torch.no_grad():
        y = m.to(dev)(x.to(dev))
    assert_close(y, ref, torch.float32, f"model L={L}")


def test_forward_graph_replays_match_eager(dev):
    """Every replay of a recorded LM forward (padded length, side-stream fork/join in every
    block) equals the eager forward on the same ids; eager work and synchronisations run
    between the replays, and a replay after a weight update in place sees the new weight."""
    print("forward graph", flush=True)
    lm = make_lm("lm_c3", n_layers=2).to(torch.bfloat16).to(dev)
    ids = [lm_input("lm_c3", B=2, L=200, seed=s).to(dev) for s in (1, 2, 3)]
    with torch.no_grad():
        fg = lm.capture_forward(ids[0])
        for rep in range(6):
            x = ids[rep % 3]
            want = lm(x)
            torch.cuda.synchronize()
            got = fg(x).clone()
            torch.cuda.synchronize()
            err = max_rel(got, want)
            print("  replay", rep, "max rel vs eager", err, flush=True)
            assert err < 1e-3, f"replay {rep}: {err}"
        lm.backbone.layers[1].out_proj.weight.mul_(0.5)
        want = lm(ids[0])
        got = fg(ids[0]).clone()
        assert max_rel(got, want) < 1e-3
    with pytest.raises(RuntimeError):
        fg(ids[0][:, :100])


@pytest.mark.parametrize("name", ["lm_c3", "lm_c4"])
def test_block_at_lm_shape(dev, name):
    """One block at the full shape of the 12-layer (d_model 768, 12 heads, B=8, L=4096) and
    the 24-layer long-context (d_model 1024, d_state 128, 16 heads, B=1, L=32768) models,
    with decays drawn from U[0.9, 0.999] so the scan and slot carries span many chunks."""
    from hdcmamba_amd import HdcMamba9v3Block
    from cfgs import reinit_block_

    cfg = WORKLOADS[name]
    print("block at", name, cfg["B"], cfg["L"], cfg["d_model"], flush=True)
    torch.manual_seed(11)
    blk = HdcMamba9v3Block(cfg["d_model"], cfg["d_state"], cfg["num_heads"], cfg["chunk"])
    blk = reinit_block_(blk, seed=11, decays_uniform=True).eval().to(torch.bfloat16)
    g = torch.Generator().manual_seed(12)
    x = torch.randn(cfg["B"], cfg["L"], cfg["d_model"], generator=g).to(torch.bfloat16)
    ref = oracle.block_forward(_sd(blk), x, oracle_cfg(blk))
    with torch.no_grad():
        y, _ = blk.to(dev)(x.to(dev))
    print("max rel", max_rel(y, ref), flush=True)
    assert_close(y, ref, torch.bfloat16, name)


def test_model_two_layers_long_context(dev):
    """Two layers of the long-context model (d_model 1024, d_state 128, 16 heads) over one
    sequence of 32768 tokens: residual stream, per-block norms and the final norm."""
    from hdcmamba_amd import HdcMamba9v3Model
    from cfgs import reinit_block_

    cfg = WORKLOADS["lm_c4"]
    print("model 2 layers", cfg["L"], flush=True)
    torch.manual_seed(13)
    m = HdcMamba9v3Model(cfg["d_model"], 2, cfg["d_state"], cfg["chunk"], num_heads=cfg["num_heads"],
                         chunk_size=cfg["chunk"])
    for i, blk in enumerate(m.layers):
        reinit_block_(blk, seed=20 + i, decays_uniform=True)
    m = m.eval().to(torch.bfloat16)
    x = torch.randn(1, cfg["L"], cfg["d_model"], generator=torch.Generator().manual_seed(14)).to(torch.bfloat16)
    ref = oracle.model_forward(_sd(m), x, oracle.BlockCfg(cfg["d_model"], cfg["d_state"], cfg["num_heads"],
                                                          cfg["chunk"]), 2)
    with torch.no_grad():
        y = m.to(dev)(x.to(dev))
    print("max rel", max_rel(y, ref), flush=True)
    assert_close_normwise(y, ref, torch.bfloat16, "2-layer model L=32768")


def test_empty_inputs(dev):
    """Zero-length sequences and empty batches run through the block, the model and the LM
    (no kernel touches the empty buffers) and give empty outputs of the right shape; the
    LN+conv backward of an empty input gives zero parameter gradients."""
    from hdcmamba_amd import FusedNormConv1dFunction, HdcMamba9v3Block, HdcMamba9v3Model, HdcMambaLM

    print("empty inputs", flush=True)
    torch.manual_seed(0)
    blk = HdcMamba9v3Block(256, 64, 4, 64).to(dev).eval()
    for shape in ((2, 0, 256), (0, 64, 256)):
        with torch.no_grad():
            y, _ = blk(torch.zeros(shape, device=dev))
        assert tuple(y.shape) == shape
    m = HdcMamba9v3Model(256, 2, 64, 32, num_heads=4, chunk_size=64).to(dev).eval()
    with torch.no_grad():
        assert tuple(m(torch.zeros(1, 0, 256, device=dev)).shape) == (1, 0, 256)
    lm = HdcMambaLM(256, 1, 64, 4, vocab_size=128, chunk_size=64).to(dev).eval()
    with torch.no_grad():
        assert tuple(lm(torch.zeros(1, 0, dtype=torch.long, device=dev)).shape) == (1, 0, 128)
    x = torch.zeros(2, 0, 256, device=dev, requires_grad=True)
    w = torch.ones(256, device=dev, requires_grad=True)
    b = torch.zeros(256, device=dev, requires_grad=True)
    cw = torch.randn(256, 4, device=dev, requires_grad=True)
    cb = torch.zeros(256, device=dev, requires_grad=True)
    FusedNormConv1dFunction.apply(x, w, b, cw, cb, 1e-5).sum().backward()
    for t in (w, b, cw, cb):
        assert t.grad is not None and t.grad.abs().max().item() == 0.0
    # a non-empty sum: its gradient reaches the backward as an expanded (stride-0) tensor
    x = torch.randn(2, 5, 256, device=dev, requires_grad=True)
    FusedNormConv1dFunction.apply(x, w, b, cw, cb, 1e-5).sum().backward()
    xr = x.detach().cpu().requires_grad_(True)
    ref = oracle.norm_conv(xr, w.detach().cpu(), b.detach().cpu(), cw.detach().cpu(), cb.detach().cpu(), 1e-5)
    ref.sum().backward()
    assert max_rel(x.grad, xr.grad) <= 1e-4


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name", ["lm_c3", "lm_c4"])
def test_lm_logits_against_oracle(dev, name):
    """The whole headline LM end to end in bf16 (12 layers d_model 768 at B=8 x 4096, and 24
    layers d_model 1024 d_state 128 at B=1 x 32768; vocab 50304, default init) against the
    oracle's LM forward (the whole backbone on the CPU): the head's input (norm_f's output) at
    every position, and the logits at 64 positions per sequence (the last 16 and 48 drawn at
    random), normwise."""
    cfg = WORKLOADS[name]
    print("lm end to end", name, flush=True)
    lm = make_lm(name, seed=5).to(torch.bfloat16)
    ids = lm_input(name, seed=6)
    L = ids.shape[1]
    g = torch.Generator().manual_seed(7)
    pos = sorted(set(torch.randint(0, L - 16, (48,), generator=g).tolist()) | set(range(L - 16, L)))
    seen = {}
    hook = lm.lm_head.register_forward_pre_hook(lambda m, a: seen.__setitem__("h", a[0].float().cpu()))
    try:
        with torch.no_grad():
            logits = lm.to(dev)(ids.to(dev))
    finally:
        hook.remove()
    got = logits[:, pos].float().cpu()
    del logits
    torch.cuda.empty_cache()
    ref, ref_h = oracle.lm_forward(_sd(lm), ids, oracle.BlockCfg(cfg["d_model"], cfg["d_state"], cfg["num_heads"],
                                                                 cfg["chunk"]), cfg["n_layers"], positions=pos,
                                   return_hidden=True)
    print("hidden max rel", max_rel(seen["h"], ref_h), "logits max rel", max_rel(got, ref), flush=True)
    assert seen["h"].shape == ref_h.shape
    assert_close_normwise(seen["h"], ref_h, torch.bfloat16, f"{name} head input, every position")
    assert_close_normwise(got, ref, torch.bfloat16, f"{name} logits")

