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


def test_close_restores_the_modules_settings():
    """The decoder switches its MLAs to absolute RoPE positions and (for
    graph replays) the per-row split plan; close() / the with-block undoes
    both."""
    a, b = _mla(), _mla()
    a.rope_positions, a.split_plan = "chunk", "auto"
    m = TinyModel(64, 256, 64, [a, b])
    before = [(x.rope_positions, x.split_plan) for x in (a, b)]
    with IncrementalDecoder(m) as dec:
        for x in dec.mlas:
            x.rope_positions, x.split_plan = "absolute", "static"  # what prefill() / the capture set
    assert [(x.rope_positions, x.split_plan) for x in (a, b)] == before


def test_positions_bounded_by_the_smallest_cache():
    """A step past the shortest MLA cache raises on the host before anything
    runs, eager or replayed (the kernels would skip the append and only set a
    device flag)."""
    m = TinyModel(64, 256, 64, [_mla(), _mla()])
    dec = IncrementalDecoder(m)
    dec.limit, dec.pos = 40, 39
    dec._check_room(1)
    with pytest.raises(ValueError, match="smallest MLA cache length"):
        dec._check_room(2)
