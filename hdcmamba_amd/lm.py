"""Language-model wrapper around HdcMamba9v3Model (embedding -> backbone -> norm_f -> tied head).

Mirrors the HdcMamba arm of the reference harness's ``UniversalLM``
(train_fineweb.py:23-94): ``nn.Embedding`` -> ``HdcMamba9v3Model`` (which ends in its own
``norm_final``) -> ``norm_f`` LayerNorm -> ``lm_head`` tied to the embedding.  The
construction order (embedding, backbone, norm_f, lm_head, then normal(0, 0.04) on the
embedding and again on the tied head, LayerNorm to ones/zeros) follows
train_fineweb.py:49-84 so seeded construction draws the same weights.
"""
from __future__ import annotations

import copy

import torch
import torch.nn as nn

from . import _ops
from .model import BlockState, HdcMamba9v3Model, layer_norm

__all__ = ["HdcMambaLM", "DecodeGraph", "ForwardGraph", "SIZES"]

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
        # the embedding output is this forward's own; norm_f follows norm_final (fused in inference)
        x = self.backbone._forward(x, owned=True, then=self.norm_f)
        return self.lm_head(x)

    def _logits(self, x):
        """norm_f then the tied head.  The head stays on the library GEMM even for the few
        rows of a decode step: at V=50304 it streams 206 MB and hipBLASLt's skinny solution
        runs it in about 48 us against 55 us on the skinny decode kernel."""
        x = layer_norm(x, self.norm_f.weight, self.norm_f.bias, self.norm_f.eps)
        return self.lm_head(x)

    def prefill(self, input_ids, last=1):
        """Forward over input_ids [B,L] returning the logits of the last ``last`` positions
        ([B,last,V]) and the per-block states for ``step``."""
        _ops._on_gpu(input_ids)
        with torch.no_grad():
            y, states = self.backbone.prefill(self.embedding(input_ids))
            return self._logits(y[:, y.shape[1] - last:]), states

    def step(self, input_ids, states, pos_dev=None):
        """One token per batch row: input_ids [B] -> logits [B,V]; states advance in place."""
        _ops._on_gpu(input_ids)
        with torch.no_grad():
            # the embedding rows by indexing (PyTorch's gather kernel: ~2 us for 16 rows against
            # ~7 us for nn.Embedding's index_select kernel, the same rows); norm_final and norm_f
            # in one pass, then the tied head
            x = self.embedding.weight[input_ids]
            return self.lm_head(self.backbone.step(x, states, pos_dev, then=self.norm_f))

    def capture_decode(self, states):
        """A DecodeGraph stepping ``states`` (as returned by prefill) from replays."""
        return DecodeGraph(self, states)

    def capture_forward(self, input_ids):
        """A ForwardGraph replaying this model's inference forward at input_ids' shape."""
        return ForwardGraph(self, input_ids)


def _clone_state(st):
    return BlockState(conv=st.conv.clone(), h=st.h.clone(), S_prev=st.S_prev.clone(),
                      S_intra=st.S_intra.clone(), pos=st.pos)


class DecodeGraph:
    """One decode step of an HdcMambaLM recorded once as a HIP graph and replayed per token.

    The graph reads token ids from a static buffer, runs embedding -> every block's step ->
    norm_final -> norm_f -> lm_head into a static logits buffer, and advances a device-side
    chunk offset that every block's mixer step reads, so one recording serves every
    position.  A replay submits the whole step (three kernels per block at d_model >= 512 in
    bf16: the LayerNorm + conv + in_proj front, the mixer step and out_proj) at once instead
    of launching each from Python.  The states passed in are the ones the replays
    update; ``step`` keeps their host-side ``pos`` in sync.  Replays of one DecodeGraph must
    not overlap with other work on the same states.
    """

    def __init__(self, lm, states):
        chunks = {layer.chunk_size for layer in lm.backbone.layers}
        pos = {st.pos for st in states}
        if len(chunks) != 1 or len(pos) != 1 or len(states) != len(lm.backbone.layers):
            raise RuntimeError("capture_decode needs one chunk size and states at one position")
        (self.chunk,) = chunks
        self.lm, self.states = lm, states
        dev = states[0].h.device
        B = states[0].h.shape[0]
        self.ids = torch.zeros(B, dtype=torch.long, device=dev)
        self.pos = torch.full((1,), states[0].pos, dtype=torch.int32, device=dev)
        # warm up on scratch copies (library handles, allocator pools), then record
        scratch = [_clone_state(st) for st in states]
        scratch_pos = self.pos.clone()
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(2):
                self._run(scratch, scratch_pos)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        del scratch, scratch_pos
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = self._run(self.states, self.pos)

    def _run(self, states, pos):
        with torch.no_grad():
            logits = self.lm.step(self.ids, states, pos_dev=pos)
            _ops.chunk_pos_advance(pos, self.chunk)
        return logits

    def step(self, input_ids):
        """input_ids [B] -> logits [B,V] (a static buffer, overwritten by the next step)."""
        self.ids.copy_(input_ids)
        self.graph.replay()
        for st in self.states:
            st.pos = (st.pos + 1) % self.chunk
        return self.logits


class ForwardGraph:
    """The inference forward of an HdcMambaLM at one input shape, recorded once as a HIP
    graph and replayed per call.

    A forward at B=1, L=32768 issues about 170 kernels (seven per block); launched one by
    one from Python they leave the GPU idle between launches (eager forwards ~15.6 ms against
    ~14.2 ms replayed).
    A replay submits the recorded sequence at once, including the side-stream fork and
    join of every block.  ``forward(input_ids)`` copies the ids into the static input
    buffer and returns the static logits buffer, which the next replay overwrites.  The
    weights are read at replay time (in place updates are seen: values derived from a
    weight and kept between forwards, the out_proj row sums, are refreshed in place before
    a replay when the weight's version changed); the recorded shapes, dtypes and buffers
    are fixed.
    """

    def __init__(self, lm, input_ids, warmup=2):
        _ops._on_gpu(input_ids)
        if lm.training:
            raise RuntimeError("capture_forward records the inference forward; call eval() first")
        dev = input_ids.device
        self.lm = lm
        self.ids = input_ids.detach().clone()
        # warm library handles and allocator pools outside the recording
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(warmup):
                lm(self.ids)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph):
            self.logits = lm(self.ids)
        self._refresh = [m for m in lm.modules() if hasattr(m, "refresh_derived_weights")]

    def forward(self, input_ids):
        if input_ids.shape != self.ids.shape:
            raise RuntimeError(f"ForwardGraph was recorded for ids of shape {tuple(self.ids.shape)}, "
                               f"got {tuple(input_ids.shape)}")
        with torch.no_grad():
            for m in self._refresh:
                m.refresh_derived_weights()
        self.ids.copy_(input_ids)
        self.graph.replay()
        return self.logits

    __call__ = forward
