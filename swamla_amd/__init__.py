"""swamla_amd — MI355X-native (gfx950) MLA latent-KV-cache inference path.

A drop-in for the absorb branch of Orolol/swamla's ``MLA`` module
(models/mla.py): fused cache append, absorbed split-KV decode attention and
log-sum-exp merge as hand-written HIP kernels behind a C-ABI
(include/swamla_mi355x.h), driven from PyTorch-ROCm host code.
"""
from .config import MLAConfig
from .generate import IncrementalDecoder
from .kernels import DecodeWorkspace, LatentCache, append, decode_attention, plan_splits
from .mla import MLA
from .rope import RoPE, rope_tables

__all__ = [
    "MLA",
    "MLAConfig",
    "IncrementalDecoder",
    "RoPE",
    "rope_tables",
    "LatentCache",
    "DecodeWorkspace",
    "append",
    "decode_attention",
    "plan_splits",
]
