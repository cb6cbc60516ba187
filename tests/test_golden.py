"""The oracle's restatement of the reference MLA reproduces the reference's
own outputs and caches bit-exactly (fixtures from tests/golden/make_golden.py,
written by importing Orolol/swamla models/mla.py)."""
import glob
import hashlib
import os

import pytest
import torch

from oracle.mla_ref import MLAConfig, RefMLA, enable_cache, init_weights

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "mla_*.pt")))


def checksums(module):
    """SHA-256 of each parameter's fp32 bytes (as tests/golden/make_golden.py)."""
    return {n: hashlib.sha256(p.detach().float().contiguous().numpy().tobytes()).hexdigest()
            for n, p in module.named_parameters()}


def load(path):
    return torch.load(path, weights_only=True)


def build_ref(meta):
    cfg = MLAConfig(n_embd=meta["dim"], max_batch_size=meta["batch"], max_seq_len=meta["max_seq_len"])
    m = RefMLA(cfg)
    init_weights(m, meta["seed"], ln_random=meta["ln_random"])
    return m


def test_fixtures_present():
    assert len(GOLDEN) == 6
    assert sum("masked" in os.path.basename(p) for p in GOLDEN) == 2


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_restatement_matches_reference_bitwise(path):
    blob = load(path)
    meta = blob["meta"]
    m = build_ref(meta)
    # The regenerated weights are the ones the reference ran with.
    assert checksums(m) == blob["checksums"]
    m.eval()
    enable_cache(m)
    dtype = torch.bfloat16 if "bfloat16" in meta["dtype"] else torch.float32
    m.to(dtype)
    pos = 0
    with torch.no_grad():
        masks = blob.get("masks") or [None] * len(blob["inputs"])
        for x, ref_out, mask in zip(blob["inputs"], blob["outputs"], masks):
            out = m(x, pos, None, mask)
            assert out.dtype == ref_out.dtype
            assert torch.equal(out, ref_out), f"output mismatch at start_pos={pos}"
            pos += x.shape[1]
    assert torch.equal(m.kv_cache[: meta["batch"], :pos], blob["kv_cache"])
    assert torch.equal(m.pe_cache[: meta["batch"], :pos], blob["pe_cache"])


def test_reference_set_inference_mode_quirk():
    """The reference's set_inference_mode(True) raises as constructed (plain
    None attributes vs register_buffer, mla.py:180-182 / :209); the oracle
    restates that, and enable_cache is the harness step around it."""
    m = RefMLA(MLAConfig(n_embd=64, max_batch_size=1, max_seq_len=8))
    with pytest.raises(KeyError):
        m.set_inference_mode(True)
    m2 = RefMLA(MLAConfig(n_embd=64, max_batch_size=1, max_seq_len=8))
    enable_cache(m2)
    assert m2.kv_cache.shape == (1, 8, 256) and m2.kv_cache.dtype == torch.float32
