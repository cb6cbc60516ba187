"""CPU checks of the incremental decoder's set-up (no kernel runs): it takes
models whose blocks all hold the drop-in MLA and refuses the blocks whose
state it does not carry (models/swa_mla_model.py:394-406)."""
import pytest
import torch.nn as nn

from gen_model import TinyModel
from swamla_amd import MLA, MLAConfig
from swamla_amd.generate import IncrementalDecoder


def _mla():
    return MLA(MLAConfig(n_embd=256, n_head=16, kv_lora_rank=128, max_batch_size=2, max_seq_len=64))


def test_accepts_all_mla_stack():
    m = TinyModel(64, 256, 64, [_mla(), _mla()])
    dec = IncrementalDecoder(m)
    assert len(dec.mlas) == 2 and dec.block_size == 64


def test_refuses_recurrent_and_engram_blocks():
    m = TinyModel(64, 256, 64, [_mla(), _mla()])
    m.transformer.h[1] = nn.Identity()  # stands for a GatedDeltaNet block (no .attn MLA)
    with pytest.raises(NotImplementedError, match="DeltaNet"):
        IncrementalDecoder(m)
    m = TinyModel(64, 256, 64, [_mla()])
    m.transformer.h[0].has_engram = True
    with pytest.raises(NotImplementedError, match="Engram"):
        IncrementalDecoder(m)
