"""hdcmamba_amd: the HdcMamba block forward on MI355X (gfx950) HIP kernels.

Public names match the reference package (hdcmamba/__init__.py:1-13).
"""
from .model import (
    BlockState,
    FusedNormConv1dFunction,
    HdcMamba9v3Block,
    HdcMamba9v3Model,
    fused_norm_conv1d_trainable,
    set_differentiable_mixer,
    set_fused_out_proj,
    set_fused_step_front,
)
from .lm import DecodeGraph, ForwardGraph, HdcMambaLM

__all__ = [
    "HdcMamba9v3Block",
    "HdcMamba9v3Model",
    "FusedNormConv1dFunction",
    "fused_norm_conv1d_trainable",
    "HdcMambaLM",
    "BlockState",
    "DecodeGraph",
    "ForwardGraph",
    "set_differentiable_mixer",
    "set_fused_out_proj",
    "set_fused_step_front",
]
