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
