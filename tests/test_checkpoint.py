"""Checkpoint compatibility with the reference modules (CPU only).

The reference's own constructor wrote complete block state_dicts into the golden vectors
(tests/golden/make_golden.py runs hdcmamba/model.py:300-329); a checkpoint of the reference
must load into the build's modules with strict key and shape checking, at block, model
(model.py:396-400) and LM level (the harness LM of train_fineweb.py:49-55: embedding,
backbone, norm_f and the lm_head tied to the embedding).
"""
import io
from pathlib import Path

import pytest
import torch

from hdcmamba_amd import HdcMamba9v3Block, HdcMamba9v3Model, HdcMambaLM

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_vectors.pt"


@pytest.fixture(scope="module")
def ctors():
    d = torch.load(GOLDEN, weights_only=True)
    return [d[k] for k in sorted(d) if k.startswith("ctor_")]


def _block_sd(entry):
    return {k: v for k, v in entry.items() if k != "args"}


def test_reference_block_checkpoint_loads_strictly(ctors):
    for entry in ctors:
        dm, ds, H, C, _ = (int(v) for v in entry["args"])
        blk = HdcMamba9v3Block(dm, ds, H, C)
        sd = _block_sd(entry)
        assert set(blk.state_dict()) == set(sd)
        blk.load_state_dict(sd, strict=True)
        for k, v in sd.items():
            assert torch.equal(blk.state_dict()[k], v), k


def test_reference_model_checkpoint_loads_strictly(ctors):
    entry = ctors[0]
    dm, ds, H, C, _ = (int(v) for v in entry["args"])
    n = 3
    sd = {f"layers.{i}.{k}": v for i in range(n) for k, v in _block_sd(entry).items()}
    sd["norm_final.weight"] = torch.randn(dm)
    sd["norm_final.bias"] = torch.randn(dm)
    m = HdcMamba9v3Model(dm, n, ds, 32, num_heads=H, chunk_size=C)
    assert set(m.state_dict()) == set(sd)
    m.load_state_dict(sd, strict=True)
    assert torch.equal(m.norm_final.bias, sd["norm_final.bias"])


def test_lm_checkpoint_keys_and_tied_head_round_trip(ctors):
    entry = ctors[0]
    dm, ds, H, C, _ = (int(v) for v in entry["args"])
    V, n = 97, 2
    lm = HdcMambaLM(dm, n, ds, H, vocab_size=V, chunk_size=C)
    keys = set(lm.state_dict())
    block_keys = set(_block_sd(entry))
    want = {"embedding.weight", "lm_head.weight", "norm_f.weight", "norm_f.bias",
            "backbone.norm_final.weight", "backbone.norm_final.bias"}
    want |= {f"backbone.layers.{i}.{k}" for i in range(n) for k in block_keys}
    assert keys == want
    assert lm.lm_head.weight is lm.embedding.weight
    buf = io.BytesIO()
    torch.save(lm.state_dict(), buf)
    buf.seek(0)
    lm2 = HdcMambaLM(dm, n, ds, H, vocab_size=V, chunk_size=C)
    lm2.load_state_dict(torch.load(buf, weights_only=True), strict=True)
    assert lm2.lm_head.weight is lm2.embedding.weight
    for k, v in lm.state_dict().items():
        assert torch.equal(lm2.state_dict()[k], v), k
