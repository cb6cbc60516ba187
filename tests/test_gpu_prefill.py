"""GPU parity of mla_prefill_attn (causal attention of a prefill chunk, four
queries per workgroup) against a torch fp32 restatement of the absorbed
attention and against the per-row decode kernel on the same inputs.

Bar: the north-star bf16 tolerance, 2e-2 relative / 1e-2 absolute, against
the fp32 reference.  Chunks cover T not a multiple of four (surplus waves),
tile-boundary lengths, start positions 0 and > 0, chunk-local and absolute
RoPE, bf16 and e4m3 caches, rows clamped at the cache end, a negative start
position and sequences past the cache's batch (zero output, as decode).
"""
import pytest
import torch

from oracle import latent_ops as lo
from swamla_amd import kernels
from swamla_amd.kernels import LatentCache
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


def make_cache(B, S, fp8, gen, device, rank=R):
    """Latent rows of R_pad channels, zero beyond the rank (as the append writes them)."""
    rp = kernels.padded_rank(rank)
    c = torch.zeros(B * S, rp, device=device, dtype=torch.bfloat16)
    c[:, :rank] = torch.randn(B * S, rank, generator=gen, device=device).to(torch.bfloat16)
    if fp8:
        codes, scale = lo.fp8_quantize(c)
        return LatentCache(codes.view(B, S, rp), torch.randn(B, S, P, generator=gen, device=device).to(torch.bfloat16),
                           scale.view(B, S).float(), rank)
    return LatentCache(c.view(B, S, rp), torch.randn(B, S, P, generator=gen, device=device).to(torch.bfloat16),
                       rank=rank)


def reference(q_abs, q_pe, cos, sin, cache, sp, T, rope_abs):
    """fp32 absorbed attention per row: row r = token t of sequence b attends
    to [0, min(sp_b + t + 1, S)); empty rows (and sequences past the cache's
    batch) are zero."""
    rows = q_abs.shape[0]
    Bc, S = cache.ckv.shape[0], cache.ckv.shape[1]
    rk = cache.rank
    out = torch.zeros(rows, H, cache.rank_pad, dtype=torch.float32, device=q_abs.device)
    cos_c, sin_c = cos.cpu(), sin.cpu()
    for r in range(rows):
        b, t = divmod(r, T)
        if b >= Bc:
            continue
        L = min(int(sp[b]) + t + 1, S)
        if L <= 0:
            continue
        rp = int(sp[b]) + t if rope_abs else t
        rp = min(max(rp, 0), cos_c.shape[0] - 1)
        qpe = lo.rope_interleaved(q_pe[r:r + 1].cpu(), cos_c[rp:rp + 1][:, None], sin_c[rp:rp + 1][:, None])[0]
        if cache.scale is not None:
            c = lo.fp8_dequantize(cache.ckv[b, :L], cache.scale[b, :L])
        else:
            c = cache.ckv[b, :L].float()
        s = (q_abs[r, :, :rk].float() @ c[:, :rk].T + qpe.to(q_abs.device).float() @ cache.kpe[b, :L].float().T) * SCALE
        out[r] = torch.softmax(s, dim=-1) @ c
    return out


def check(out, ref):
    out, ref = out.float(), ref.float()
    err = (out - ref).abs()
    bad = err > 1e-2 + 2e-2 * ref.abs()
    assert not bool(bad.any()), f"{int(bad.sum())}/{bad.numel()} outside tol; max err {float(err.max()):.3e}"


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "fp8"])
@pytest.mark.parametrize("B,T,starts", [
    (1, 8, [0]),
    (2, 5, [0, 61]),
    (3, 64, [0, 1, 130]),
    (2, 65, [63, 700]),
    (1, 130, [2000]),
])
@pytest.mark.parametrize("rope_abs", [False, True], ids=["chunk", "abs"])
def test_prefill_matches_fp32_reference(gpu, fp8, B, T, starts, rope_abs):
    _prefill_case(gpu, fp8, B, T, starts, rope_abs, R)


@pytest.mark.parametrize("rank", [1, 64, 100, 173, 192])
@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "fp8"])
def test_prefill_any_rank(gpu, fp8, rank):
    """kv_lora_rank up to 256 other than 256 (padded rows; query padding ignored)."""
    _prefill_case(gpu, fp8, 2, 65, [63, 700], True, rank)


def _prefill_case(gpu, fp8, B, T, starts, rope_abs, rank):
    say(f"prefill fp8={fp8} B={B} T={T} starts={starts} rope_abs={rope_abs} rank={rank}")
    gen = torch.Generator(device=gpu).manual_seed(100 + B * 7 + T + rank)
    S = 2304
    rp = kernels.padded_rank(rank)
    cache = make_cache(B, S, fp8, gen, gpu, rank)
    cos, sin = tables(S, gpu)
    rows = B * T
    q_abs = (0.3 * torch.randn(rows, H, rp, generator=gen, device=gpu)).to(torch.bfloat16)
    q_pe = (0.3 * torch.randn(rows, H, P, generator=gen, device=gpu)).to(torch.bfloat16)
    sp = torch.tensor(starts, dtype=torch.int32, device=gpu)
    out = torch.full((rows, H, rp), float("nan"), dtype=torch.bfloat16, device=gpu)
    kernels.prefill_attention(q_abs, q_pe, cos, sin, cache, SCALE, start_pos=sp, rows_per_seq=T,
                              rope_abs=rope_abs, out=out)
    # the per-row decode kernel on the same rows (one split)
    dec = kernels.decode_attention(q_abs, q_pe, cos, sin, cache, SCALE, start_pos=sp, rows_per_seq=T,
                                   rope_abs=rope_abs, n_splits=1, min_chunk=64)
    torch.cuda.synchronize()
    ref = reference(q_abs, q_pe, cos, sin, cache, sp.cpu(), T, rope_abs)
    check(out, ref)
    check(dec, ref)


@pytest.mark.parametrize("T", [13, 14, 16])
def test_prefill_persistent_items_deterministic(gpu, T):
    """More query groups than CUs (each persistent workgroup takes several, in
    snake order), partial last groups (T not a multiple of 8: surplus columns
    repeat the last query and store its row again): three launches give the
    same bits, and the rows match the per-row decode kernel."""
    say(f"prefill persistent items T={T}")
    gen = torch.Generator(device=gpu).manual_seed(500 + T)
    B, S = 300, 640
    cache = make_cache(B, S, False, gen, gpu)
    cos, sin = tables(S, gpu)
    rows = B * T
    q_abs = (0.3 * torch.randn(rows, H, R, generator=gen, device=gpu)).to(torch.bfloat16)
    q_pe = (0.3 * torch.randn(rows, H, P, generator=gen, device=gpu)).to(torch.bfloat16)
    sp = torch.randint(0, S - T, (B,), generator=gen, device=gpu, dtype=torch.int32)
    outs = []
    for _ in range(3):
        out = torch.full((rows, H, R), float("nan"), dtype=torch.bfloat16, device=gpu)
        kernels.prefill_attention(q_abs, q_pe, cos, sin, cache, SCALE, start_pos=sp, rows_per_seq=T, out=out)
        outs.append(out)
    dec = kernels.decode_attention(q_abs, q_pe, cos, sin, cache, SCALE, start_pos=sp, rows_per_seq=T, n_splits=1,
                                   min_chunk=64)
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))
    check(outs[0], dec)


def test_prefill_edges_clamp_negative_and_past_batch(gpu):
    """Rows past the cache end are clamped to it, a negative start gives
    empty rows (zeros), sequences past the cache's batch give zeros; all as
    the decode kernel does."""
    gen = torch.Generator(device=gpu).manual_seed(7)
    Bc, S, T = 2, 300, 12
    cache = make_cache(Bc, S, False, gen, gpu)
    cos, sin = tables(S, gpu)
    sp = torch.tensor([295, -20, 4], dtype=torch.int32, device=gpu)  # third sequence: no cache row
    rows = 3 * T
    q_abs = (0.3 * torch.randn(rows, H, R, generator=gen, device=gpu)).to(torch.bfloat16)
    q_pe = (0.3 * torch.randn(rows, H, P, generator=gen, device=gpu)).to(torch.bfloat16)
    out = kernels.prefill_attention(q_abs, q_pe, cos, sin, cache, SCALE, start_pos=sp, rows_per_seq=T)
    dec = kernels.decode_attention(q_abs, q_pe, cos, sin, cache, SCALE, start_pos=sp, rows_per_seq=T,
                                   n_splits=1, min_chunk=64)
    torch.cuda.synchronize()
    ref = reference(q_abs, q_pe, cos, sin, cache, sp.cpu(), T, False)
    check(out, ref)
    check(dec, ref)
    assert bool((out[T:].float() == 0).all())  # negative start and past-batch rows


def test_prefill_partly_empty_query_group_has_no_nan(gpu):
    """A start position of -3: the first three queries of the sequence see no
    token while the others in their workgroup do; they come out zero (not
    NaN), as the decode kernel gives."""
    gen = torch.Generator(device=gpu).manual_seed(8)
    Bc, S, T = 2, 128, 12
    cache = make_cache(Bc, S, False, gen, gpu)
    cos, sin = tables(S, gpu)
    sp = torch.tensor([-3, 10], dtype=torch.int32, device=gpu)
    rows = Bc * T
    q_abs = (0.3 * torch.randn(rows, H, R, generator=gen, device=gpu)).to(torch.bfloat16)
    q_pe = (0.3 * torch.randn(rows, H, P, generator=gen, device=gpu)).to(torch.bfloat16)
    out = kernels.prefill_attention(q_abs, q_pe, cos, sin, cache, SCALE, start_pos=sp, rows_per_seq=T)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all())
    assert bool((out[:3].float() == 0).all())
    check(out, reference(q_abs, q_pe, cos, sin, cache, sp.cpu(), T, False))


def test_module_prefill_chunk_uses_prefill_kernel_and_matches_row_path(gpu, monkeypatch):
    """A 2 x 512-token bf16 prefill through MLA.forward runs mla_prefill_attn
    and agrees with the same module forced onto the per-row decode path."""
    from swamla_amd import MLA, MLAConfig

    cfg = MLAConfig(n_embd=1024, max_batch_size=2, max_seq_len=1024)
    torch.manual_seed(8)
    outs = {}
    for use in (True, False):
        m = MLA(cfg)
        g = torch.Generator().manual_seed(9)
        with torch.no_grad():
            for name, p in m.named_parameters():
                if name.endswith("weight") and not name.startswith("kv_norm"):
                    p.copy_(torch.randn(p.shape, generator=g) * 0.02)
        m.eval().to(torch.bfloat16).to(gpu)
        m.set_inference_mode(True)
        calls = []
        real = kernels.prefill_attention

        def spy(*a, **k):
            calls.append(1)
            return real(*a, **k)

        monkeypatch.setattr(kernels, "prefill_attention", spy)
        monkeypatch.setattr(kernels, "use_prefill", (lambda *a, **k: True) if use else (lambda *a, **k: False))
        gd = torch.Generator(device=gpu).manual_seed(10)
        x = torch.randn(2, 512, 1024, generator=gd, device=gpu).to(torch.bfloat16)
        with torch.no_grad():
            m(torch.randn(2, 64, 1024, generator=gd, device=gpu).to(torch.bfloat16), 0)
            outs[use] = m(x, 64)
        torch.cuda.synchronize()
        assert (len(calls) > 0) == use
    check(outs[True], outs[False])
