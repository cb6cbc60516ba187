"""Configuration object for the drop-in ``MLA``.

The reference builds a per-block dataclass from its model config
(models/swa_mla_model.py:555-606) and ``MLA.__init__`` reads the fields below
from it (models/mla.py:75-170).  ``MLA`` accepts that object, or this one,
unchanged; the two extra fields select this build's cache format and RoPE
position convention.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional


@dataclass
class MLAConfig:
    n_embd: int = 1024
    n_head: int = 16
    q_lora_rank: int = 0
    kv_lora_rank: int = 256
    qk_nope_head_dim: int = 128
    qk_rope_head_dim: int = 64
    v_head_dim: int = 128
    max_batch_size: int = 8  # mla.py:130
    max_seq_len: int = 4096  # mla.py:131 (the model passes block_size)
    dropout: float = 0.0
    bias: bool = False
    attn_impl: str = "absorb"
    rope_factor: float = 1.0
    mscale: float = 1.0
    # this build only: None / "model" keeps the cache in the module dtype,
    # "fp8_e4m3" stores e4m3 latents with one fp32 scale per token
    kv_cache_dtype: Optional[str] = None
    # this build only: "chunk" rotates by the position within the call, as
    # the reference does (positional_encoding.py:49-50); "absolute" by the
    # cache position
    rope_positions: str = "chunk"
