"""Language-model wrapper around HdcMamba9v3Model (embedding -> backbone -> norm_f -> tied head).

Mirrors the HdcMamba arm of the reference harness's ``UniversalLM``
(train_fineweb.py:23-94): ``nn.Embedding`` -> ``HdcMamba9v3Model`` (which ends in its own
``norm_final``) -> ``norm_f`` LayerNorm -> ``lm_head`` tied to the embedding.  The
construction order (embedding, backbone, norm_f, lm_head, then normal(0, 0.04) on the
embedding and again on the tied head, LayerNorm to ones/zeros) follows
train_fineweb.py:49-84 so seeded construction draws the same weights.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _ops
from .model import HdcMamba9v3Model

__all__ = ["HdcMambaLM", "SIZES"]

# HdcMamba rows of the reference size table (train_fineweb.py:29-45).
SIZES = {
    "130M": {"d_model": 768, "n_layers": 34, "d_state": 64, "num_heads": 12},
    "360M": {"d_model": 1024, "n_layers": 57, "d_state": 128, "num_heads": 16},
    "1B": {"d_model": 2048, "n_layers": 42, "d_state": 128, "num_heads": 32},
}


class HdcMambaLM(nn.Module):
    def __init__(self, d_model, n_layers, d_state, num_heads, vocab_size=50277, chunk_size=256,
                 num_slots=32):
        super().__init__()
        self.d_model = d_model
        self.embedding = nn.Embedding(vocab_size, d_model)
        self.backbone = HdcMamba9v3Model(d_model=d_model, n_layers=n_layers, d_state=d_state,
                                         num_slots=num_slots, num_heads=num_heads, chunk_size=chunk_size)
        self.norm_f = nn.LayerNorm(d_model)
        self.lm_head = nn.Linear(d_model, vocab_size, bias=False)
        self.lm_head.weight = self.embedding.weight
        for m in (self.embedding, self.lm_head, self.norm_f):
            self._init_weights(m)

    @staticmethod
    def _init_weights(module):
        if isinstance(module, (nn.Linear, nn.Embedding)):
            nn.init.normal_(module.weight, mean=0.0, std=0.04)
            if getattr(module, "bias", None) is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.LayerNorm):
            nn.init.zeros_(module.bias)
            nn.init.ones_(module.weight)

    @classmethod
    def from_size(cls, size, vocab_size=50277, chunk_size=256):
        return cls(vocab_size=vocab_size, chunk_size=chunk_size, **SIZES[size])

    def forward(self, input_ids):
        _ops._on_gpu(input_ids)
        x = self.embedding(input_ids)
        x = self.backbone(x)
        x = _ops.layer_norm(x, self.norm_f.weight, self.norm_f.bias, self.norm_f.eps)
        return self.lm_head(x)
