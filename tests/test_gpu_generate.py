"""GPU parity of model-level incremental decoding (swamla_amd.generate)
against the reference's way of generating: the whole context re-run from
position 0 for every token (models/swa_mla_model.py:507-552,
inference.py:97-102), here by the same model built on the oracle's RefMLA on
the CPU.  Teacher-forced logits at every step, and greedy generation.

Bar: fp32 logits within 1e-3 (the two sides differ only in summation order);
bf16 within 2e-2 relative / 5e-2 absolute of the fp32 reference (each layer's
bf16 roundings compound through the MLPs and lm_head; the weights are
bf16 values on both sides).
"""
import pytest
import torch

from gen_model import TinyModel
from oracle.mla_ref import MLAConfig as RefConfig
from oracle.mla_ref import RefMLA, init_weights
from swamla_amd import MLA, MLAConfig
from swamla_amd.generate import IncrementalDecoder

pytestmark = pytest.mark.gpu

V, D, S, NL = 320, 256, 64, 2


def say(*a):
    print(*a, flush=True)


def make_models(seed, dtype, gpu):
    cfg = dict(n_embd=D, n_head=16, kv_lora_rank=128, max_batch_size=2, max_seq_len=S)
    refs = []
    for i in range(NL):
        r = RefMLA(RefConfig(**cfg))
        init_weights(r, seed + i, ln_random=True)
        refs.append(r)
    ref = TinyModel(V, D, S, refs)
    g = torch.Generator().manual_seed(seed + 100)
    with torch.no_grad():
        for name, p in ref.named_parameters():
            if ".attn." in name:
                continue
            if name.endswith("norm.weight") or name.endswith("ln_f.weight"):
                p.copy_(1 + 0.1 * torch.randn(p.shape, generator=g))
            else:
                p.copy_(0.05 * torch.randn(p.shape, generator=g))
        for p in ref.parameters():  # bf16-representable, so the bf16 model holds the same weights
            p.copy_(p.to(torch.bfloat16).float())
    ref.eval()
    ours = TinyModel(V, D, S, [MLA(MLAConfig(**cfg)) for _ in range(NL)])
    ours.load_state_dict(ref.state_dict())
    ours.eval().to(dtype).to(gpu)
    return ref, ours


@pytest.mark.parametrize("graph", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_incremental_logits_match_full_recompute(gpu, dtype, graph):
    """Teacher-forced steps, eager or replayed from the captured HIP graph
    (which advances the positions on the device)."""
    say(f"incremental decoding dtype={dtype} graph={graph}")
    ref, ours = make_models(5, dtype, gpu)
    g = torch.Generator().manual_seed(6)
    toks = torch.randint(0, V, (2, 20), generator=g)
    dec = IncrementalDecoder(ours, graph=graph)
    rtol, atol = (0.0, 1e-3) if dtype == torch.float32 else (2e-2, 5e-2)
    with torch.no_grad():
        logits = [dec.prefill(toks[:, :12].to(gpu))]
        for t in range(12, 20):
            logits.append(dec.step(toks[:, t:t + 1].to(gpu)))
        torch.cuda.synchronize()
        for i, got in enumerate(logits):
            want = ref.full_logits(toks[:, :12 + i])
            err = (got.double().cpu() - want.double()).abs()
            bad = err > atol + rtol * want.double().abs()
            assert not bool(bad.any()), f"step {i}: max err {float(err.max()):.3e}"


def test_greedy_generation_matches_reference(gpu):
    say("greedy generation fp32")
    ref, ours = make_models(7, torch.float32, gpu)
    g = torch.Generator().manual_seed(8)
    prompt = torch.randint(0, V, (2, 9), generator=g)
    with torch.no_grad():
        out = IncrementalDecoder(ours).generate(prompt.to(gpu), max_new_tokens=12, top_k=1).cpu()
        want = prompt
        for _ in range(12):
            nxt = ref.full_logits(want).argmax(-1, keepdim=True)
            want = torch.cat([want, nxt], 1)
    assert torch.equal(out, want)
