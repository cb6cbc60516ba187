"""GPU parity of mla_decode_attn_append (the one-token decode step with the
append folded into the attention launch) against mla_append followed by
mla_decode_attn on the same inputs.

Bar: identical bits.  Both paths run the same append arithmetic and the same
attention kernel, so the caches (latent codes, scales, k_pe) and the outputs
must match exactly.  The rows cover the kernel's two append placements (rows
whose last split has few tiles append before any load; longer ones append
while the first tiles are in flight), single- and multi-split rows, a row at
position 0, a row whose position lies past the cache (skipped, error flag
set) and a negative position.
"""
import pytest
import torch

from swamla_amd import kernels
from swamla_amd.kernels import DecodeWorkspace, FusedAppend, LatentCache
from swamla_amd.rope import rope_tables

pytestmark = pytest.mark.gpu

R, P, H = 256, 64, 16
SCALE = 192 ** -0.5


def say(*a):
    print(*a, flush=True)


def tables(S, device):
    cos, sin = rope_tables(64, S)
    return (cos.to(torch.bfloat16)[0, 0, :, :32].contiguous().to(device),
            sin.to(torch.bfloat16)[0, 0, :, :32].contiguous().to(device))


# start positions: early path (0, 63, 64, 100), late path in one split
# (300, 1000), several splits (2047, 5000, 8190), past the cache (9000), -1
STARTS = [0, 63, 64, 100, 300, 1000, 2047, 5000, 8190, 9000, -1, 4096]


def make_case(gpu, fp8, seed):
    B, S = len(STARTS), 8192
    g = torch.Generator(device=gpu).manual_seed(seed)
    if fp8:
        cache = LatentCache.allocate(B, S, torch.bfloat16, gpu, fp8=True)
        cache.ckv.copy_(torch.randint(0, 0x7F, (B, S, R), generator=g, device=gpu, dtype=torch.uint8)
                        | (torch.randint(0, 2, (B, S, R), generator=g, device=gpu, dtype=torch.uint8) << 7))
        cache.scale.copy_(torch.rand(B, S, generator=g, device=gpu) * 1e-3 + 1e-4)
    else:
        cache = LatentCache.allocate(B, S, torch.bfloat16, gpu)
        cache.ckv.copy_(torch.randn(B, S, R, generator=g, device=gpu).to(torch.bfloat16))
    cache.kpe.copy_(torch.randn(B, S, P, generator=g, device=gpu).to(torch.bfloat16))
    buf = torch.randn(B, 400, generator=g, device=gpu).to(torch.bfloat16)  # strided wkv_a rows
    kv = buf[:, 40:40 + R + P]
    ln_w = (1 + 0.1 * torch.randn(R, generator=g, device=gpu)).to(torch.bfloat16)
    ln_b = (0.1 * torch.randn(R, generator=g, device=gpu)).to(torch.bfloat16)
    q_abs = (0.3 * torch.randn(B, H, R, generator=g, device=gpu)).to(torch.bfloat16)
    q_pe = (0.3 * torch.randn(B, H, P, generator=g, device=gpu)).to(torch.bfloat16)
    sp = torch.tensor(STARTS, dtype=torch.int32, device=gpu)
    return cache, kv, ln_w, ln_b, q_abs, q_pe, sp


def clone(cache):
    return LatentCache(cache.ckv.clone(), cache.kpe.clone(), None if cache.scale is None else cache.scale.clone())


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "fp8"])
@pytest.mark.parametrize("n_splits,min_chunk", [(1, 256), (8, 256), (40, 64)])
@pytest.mark.parametrize("rope_abs", [False, True], ids=["chunk", "abs"])
@pytest.mark.parametrize("merge", [True, False], ids=["merge", "partials"])
def test_fused_append_equals_append_then_decode(gpu, fp8, n_splits, min_chunk, rope_abs, merge):
    say(f"decode_attn_append fp8={fp8} n_splits={n_splits} min_chunk={min_chunk} rope_abs={rope_abs} merge={merge}")
    cache0, kv, ln_w, ln_b, q_abs, q_pe, sp = make_case(gpu, fp8, 70 + n_splits)
    cos, sin = tables(8192, gpu)
    rows = sp.numel()
    results = []
    for fused in (False, True):
        cache = clone(cache0)
        err = torch.zeros(1, dtype=torch.int32, device=gpu)
        ws = DecodeWorkspace.allocate(rows, n_splits, gpu) if n_splits > 1 else None
        if ws is not None:
            ws.o_part.fill_(float("nan"))
            ws.lse_part.fill_(float("nan"))
        out = torch.full((rows, H, R), float("nan"), dtype=torch.bfloat16, device=gpu)
        fa = None
        if fused:
            fa = FusedAppend(kv, ln_w, ln_b, 1e-5, err)
        else:
            kernels.append(kv, cache, ln_w, ln_b, 1e-5, cos, sin, start_pos=sp, tokens_per_seq=1,
                           rope_abs=rope_abs, err_flag=err)
        kernels.decode_attention(q_abs, q_pe, cos, sin, cache, SCALE, start_pos=sp, rows_per_seq=1,
                                 rope_abs=rope_abs, n_splits=n_splits, min_chunk=min_chunk, out=out,
                                 workspace=ws, merge=merge, append=fa)
        torch.cuda.synchronize()
        results.append((cache, err, out, ws))
    (c0, e0, o0, w0), (c1, e1, o1, w1) = results
    assert int(e0.item()) == 1 and int(e1.item()) == 1  # the rows at 9000 and -1
    assert torch.equal(c0.ckv, c1.ckv)
    assert torch.equal(c0.kpe, c1.kpe)
    if fp8:
        assert torch.equal(c0.scale, c1.scale)
    # the appended tokens really changed the cache
    assert not torch.equal(c0.kpe, cache0.kpe)
    # outputs: identical bits wherever the unfused path wrote them (rows left
    # to partials keep NaN in o_lat in both)
    assert torch.equal(torch.isnan(o0), torch.isnan(o1))
    assert torch.equal(torch.nan_to_num(o0), torch.nan_to_num(o1))
    if w0 is not None and not merge:
        assert torch.equal(torch.isnan(w0.o_part), torch.isnan(w1.o_part))
        assert torch.equal(torch.nan_to_num(w0.o_part), torch.nan_to_num(w1.o_part))
        assert torch.equal(torch.nan_to_num(w0.lse_part), torch.nan_to_num(w1.lse_part))


def test_fused_append_single_row_per_length(gpu):
    """One row per call at lengths around the tile and placement edges, so
    each call is a lone block stream (no other row's work hides a race)."""
    cache0, kv, ln_w, ln_b, q_abs, q_pe, _ = make_case(gpu, False, 90)
    cos, sin = tables(8192, gpu)
    for start in (0, 1, 127, 128, 191, 192, 255, 256, 257, 320, 4095):
        say(f"single row start={start}")
        outs, caches = [], []
        for fused in (False, True):
            cache = LatentCache(cache0.ckv[:1].clone(), cache0.kpe[:1].clone())
            sp = torch.tensor([start], dtype=torch.int32, device=gpu)
            fa = FusedAppend(kv[:1], ln_w, ln_b, 1e-5) if fused else None
            if not fused:
                kernels.append(kv[:1], cache, ln_w, ln_b, 1e-5, cos, sin, start_pos=sp, tokens_per_seq=1)
            outs.append(kernels.decode_attention(q_abs[:1], q_pe[:1], cos, sin, cache, SCALE, start_pos=sp,
                                                 n_splits=1, min_chunk=256, append=fa))
            caches.append(cache)
        torch.cuda.synchronize()
        assert torch.equal(caches[0].ckv, caches[1].ckv), start
        assert torch.equal(caches[0].kpe, caches[1].kpe), start
        assert torch.equal(outs[0], outs[1]), start


def test_fused_append_rejects_prefill_rows(gpu):
    cache0, kv, ln_w, ln_b, q_abs, q_pe, sp = make_case(gpu, False, 91)
    cos, sin = tables(8192, gpu)
    with pytest.raises(ValueError):
        kernels.decode_attention(q_abs[:4], q_pe[:4], cos, sin, cache0, SCALE, start_pos=sp[:2], rows_per_seq=2,
                                 append=FusedAppend(kv[:4], ln_w, ln_b, 1e-5))
