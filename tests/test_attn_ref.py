"""CPU pin of the tests' fp32 attention restatement (tests/attn_ref.py,
which the full-size GPU checks of configurations 3-5 compare against) to the
oracle's fp64 statement, oracle/latent_ops.absorbed_attention_f64
(models/mla.py:417-487 re-associated).  Ragged rows, an empty row, a
non-trivial rank and an e4m3-dequantised cache; the output to fp32 accuracy
and the log-sum-exp to 1e-5.  A wrong softmax scale, a dropped rope term and
an off-by-one length must all miss those bars."""
import pytest
import torch

from attn_ref import SCALE, ref_attention_fp32
from oracle import latent_ops as lo

H = 16


def _inputs(rows, L, R, seed, fp8=False):
    g = torch.Generator().manual_seed(seed)
    q_abs = torch.randn(rows, H, R, generator=g) * 0.3
    q_pe = torch.randn(rows, H, 64, generator=g) * 0.3
    c = torch.randn(rows, L, R, generator=g)
    p = torch.randn(rows, L, 64, generator=g)
    if fp8:
        codes, scale = lo.fp8_quantize(c.reshape(-1, R))
        c = lo.fp8_dequantize(codes, scale).view(rows, L, R)
    return q_abs, q_pe, c, p


def _f32(q_abs, q_pe, c, p, lens, scale=SCALE, cut=0):
    return ref_attention_fp32(q_abs, q_pe, lambda r, L: c[r, : L - cut], lambda r, L: p[r, : L - cut],
                              lens, scale=scale)


@pytest.mark.parametrize("R,fp8", [(256, False), (173, False), (256, True)])
def test_fp32_restatement_matches_fp64_oracle(R, fp8):
    rows, L = 5, 700
    q_abs, q_pe, c, p = _inputs(rows, L, R, R + fp8, fp8)
    lens = [700, 1, 0, 333, 64]
    o32, lse32 = _f32(q_abs, q_pe, c, p, lens)
    o64, lse64 = lo.absorbed_attention_f64(q_abs, q_pe, c, p, lens, list(range(rows)), SCALE)
    assert torch.isinf(lse32[2]).all() and (o32[2] == 0).all()  # the empty row
    live = [0, 1, 3, 4]
    err = (o32[live].double() - o64[live]).abs().max().item()
    assert err <= 2e-6, err
    lerr = (lse32[live].double() - lse64[live]).abs().max().item()
    assert lerr <= 1e-5, lerr


def test_planted_mistakes_miss_the_bars():
    rows, L, R = 3, 500, 256
    q_abs, q_pe, c, p = _inputs(rows, L, R, 9)
    lens = [500, 250, 77]
    o64, lse64 = lo.absorbed_attention_f64(q_abs, q_pe, c, p, lens, list(range(rows)), SCALE)

    def worst(o, lse):
        return (o.double() - o64).abs().max().item(), (lse.double() - lse64).abs().max().item()

    # a softmax scale of 1/sqrt(128) (the nope dim alone) instead of 1/sqrt(192)
    eo, el = worst(*_f32(q_abs, q_pe, c, p, lens, scale=128 ** -0.5))
    assert eo > 1e-3 and el > 1e-3
    # the rope term dropped
    eo, el = worst(*_f32(q_abs, torch.zeros_like(q_pe), c, p, lens))
    assert eo > 1e-3 and el > 1e-3
    # the last cached token dropped
    eo, el = worst(*ref_attention_fp32(q_abs, q_pe, lambda r, n: c[r, : n - 1], lambda r, n: p[r, : n - 1], lens))
    assert eo > 1e-4 or el > 1e-4
