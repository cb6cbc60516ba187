"""GPU parity of the three kernels against the oracle (oracle/latent_ops.py).

Bars: cache contents bit-exact (torch's CPU LayerNorm order, per-op-rounded
RoPE, torch's e4m3 cast, scatter); attention outputs within 2e-2 relative /
1e-2 absolute in bf16 (the north_star tolerance), 1e-4 in fp32.
"""
import math

import numpy as np
import pytest
import torch

from attn_ref import check_lse
from oracle import latent_ops as lo
from swamla_amd import _abi, kernels
from swamla_amd.kernels import DecodeWorkspace, LatentCache
from swamla_amd.rope import rope_tables

pytestmark = pytest.mark.gpu

R, P, H = 256, 64, 16
SCALE = 192 ** -0.5


def say(*a):
    print(*a, flush=True)


def tables(dtype, S, device):
    cos, sin = rope_tables(64, S)
    return (cos.to(dtype)[0, 0, :, :32].contiguous().to(device), sin.to(dtype)[0, 0, :, :32].contiguous().to(device))


def close(out, ref, rtol, atol):
    out, ref = out.double().cpu(), ref.double().cpu()
    err = (out - ref).abs()
    lim = atol + rtol * ref.abs()
    bad = err > lim
    assert not bool(bad.any()), f"{int(bad.sum())} / {bad.numel()} outside tol; max err {float(err.max()):.3e}"


# ------------------------------------------------------------------ append
def _append_case(gpu, dtype, fp8, n_tok=37, B=4, S=64, seed=0, rank=R, special=False):
    say(f"append case dtype={dtype} fp8={fp8} n_tok={n_tok} rank={rank} special={special}")
    rp = kernels.padded_rank(rank)
    g = torch.Generator().manual_seed(seed)
    # rows [R_pad latent | P rope] with 16 spare columns; the latent padding
    # R .. R_pad-1 holds garbage the kernel must ignore
    kv = torch.randn(n_tok, rp + P + 16, generator=g) * 2 + 0.3
    kv = kv.to(dtype)
    w = (1 + 0.1 * torch.randn(rank, generator=g)).to(dtype)
    b = (0.1 * torch.randn(rank, generator=g)).to(dtype)
    nan_rows = []
    if special:
        # non-finite rows (NaN outputs; the payload bits of a NaN are not
        # compared), a NaN in a rope pair, and channels with w = 0 whose
        # outputs are b: subnormal bf16 values, which must survive the
        # rounding unchanged
        kv[0, 3] = float("nan")
        kv[1, 10] = float("inf")
        kv[2, rp + 5] = float("nan")
        w[20:24] = 0
        b[20:24] = torch.tensor([2.0 ** -130, -2.0 ** -128, 2.0 ** -133, 3 * 2.0 ** -133]).to(dtype)
        nan_rows = [0, 1]
    seq = torch.randint(0, B, (n_tok,), generator=g, dtype=torch.int32)
    # distinct destination per token: a random permutation of the (b, pos) grid
    flat = torch.randperm(B * S, generator=g)[:n_tok]
    seq = (flat // S).to(torch.int32)
    dst = (flat % S).to(torch.int32)
    rpos = torch.randint(0, S, (n_tok,), generator=g, dtype=torch.int32)
    cache = LatentCache.allocate(B, S, dtype, gpu, fp8=fp8, rank=rank)
    canary_c = torch.randint(0, 255, cache.ckv.shape, generator=g).to(torch.uint8) if fp8 else \
        torch.randn(cache.ckv.shape, generator=g).to(dtype)
    canary_p = torch.randn(cache.kpe.shape, generator=g).to(dtype)
    cache.ckv.copy_(canary_c)
    cache.kpe.copy_(canary_p)
    if fp8:
        cache.scale.fill_(-1.0)
    cos, sin = tables(dtype, S, gpu)
    kvg = kv.to(gpu)
    kernels.append(kvg, cache, w.to(gpu), b.to(gpu), 1e-5, cos, sin,
                   seq_idx=seq.to(gpu), dst_pos=dst.to(gpu), rope_pos=rpos.to(gpu))
    torch.cuda.synchronize()

    # expected rows: torch's CPU LayerNorm over the R channels (the
    # reference's kv_norm, restated op for op by the oracle), zeros in the
    # padding
    y = lo.layernorm_aten(kv[:, :rank], w, b, 1e-5)[0]
    ref_ln = torch.nn.functional.layer_norm(kv[:, :rank], (rank,), w, b, 1e-5)
    fin = [i for i in range(n_tok) if i not in nan_rows]
    assert torch.equal(y[fin].view(torch.uint8), ref_ln[fin].view(torch.uint8)), "oracle LayerNorm differs from torch's"
    assert bool(torch.isnan(y[nan_rows]).all()) and bool(torch.isnan(ref_ln[nan_rows]).all())
    y = torch.cat([y, torch.zeros(n_tok, rp - rank, dtype=y.dtype)], 1)
    cos_c, sin_c = cos.cpu(), sin.cpu()
    kpe = lo.rope_interleaved(kv[:, rp:rp + P], cos_c[rpos.long()], sin_c[rpos.long()])
    exp_c = canary_c.clone()
    exp_p = canary_p.clone()
    if fp8:
        codes, scale = lo.fp8_quantize(y)
        exp_c[seq.long(), dst.long()] = codes
        exp_s = torch.full((B, S), -1.0)
        exp_s[seq.long(), dst.long()] = scale
        assert torch.equal(cache.scale.cpu(), exp_s), "fp8 scales differ"
    else:
        exp_c[seq.long(), dst.long()] = y
    exp_p[seq.long(), dst.long()] = kpe
    got_c, got_p = cache.ckv.cpu(), cache.kpe.cpu()
    if special:
        # NaN cells: NaN on both sides, then compared as one canonical pattern
        for t in (got_c, exp_c, got_p, exp_p):
            t[torch.isnan(t)] = float("nan")
        assert bool((cache.ckv[seq[:2].long(), dst[:2].long(), :rank].isnan()).all().item())
        assert bool(got_c[seq[2].long(), dst[2].long(), 20:24].view(torch.int16).eq(b[20:24].view(torch.int16)).all())
    if dtype == torch.float32 or fp8:
        assert torch.equal(got_c, exp_c), "latent rows differ"
    else:
        assert torch.equal(got_c.view(torch.int16), exp_c.view(torch.int16)), "latent rows differ"
    assert torch.equal(got_p.view(torch.int16) if dtype == torch.bfloat16 else got_p,
                       exp_p.view(torch.int16) if dtype == torch.bfloat16 else exp_p), "k_pe rows differ"


@pytest.mark.parametrize("dtype,fp8", [(torch.bfloat16, False), (torch.float32, False), (torch.bfloat16, True)])
def test_append_bit_exact(gpu, dtype, fp8):
    _append_case(gpu, dtype, fp8)


@pytest.mark.parametrize("rank", [1, 64, 100, 128, 173, 200, 320, 384, 449, 512, 600, 777, 1000, 1024])
@pytest.mark.parametrize("dtype,fp8", [(torch.bfloat16, False), (torch.float32, False), (torch.bfloat16, True)])
def test_append_bit_exact_any_rank(gpu, dtype, fp8, rank):
    """kv_lora_rank other than 256 (the real model scales it per layer, up to
    1024 from SWAMLAConfig's base of 512): rows padded to a multiple of 64
    channels, the padding written as zeros."""
    _append_case(gpu, dtype, fp8, rank=rank, seed=rank)


@pytest.mark.parametrize("n_tok", [37, 200])
def test_append_special_values(gpu, n_tok):
    """Non-finite rows give NaN rows, as torch's LayerNorm does; subnormal bf16
    outputs (w = 0, b subnormal) are kept bit for bit.  200 tokens take the
    grouped prompt-size kernel, 37 as well (any count uses it for aligned
    rank-256 bf16 rows)."""
    _append_case(gpu, torch.bfloat16, False, n_tok=n_tok, B=4, S=64, seed=9, special=True)


def test_append_many_tokens_bit_exact(gpu):
    _append_case(gpu, torch.bfloat16, False, n_tok=4093, B=8, S=1024, seed=3)
    _append_case(gpu, torch.bfloat16, True, n_tok=4093, B=8, S=1024, seed=4)


def test_append_out_of_range_is_skipped_and_flagged(gpu):
    say("append out-of-range")
    dtype = torch.bfloat16
    cache = LatentCache.allocate(2, 8, dtype, gpu)
    cos, sin = tables(dtype, 8, gpu)
    kv = torch.randn(3, 320, dtype=dtype, device=gpu)
    seq = torch.tensor([0, 1, 2], dtype=torch.int32, device=gpu)  # 2 >= batch
    dst = torch.tensor([0, 9, 1], dtype=torch.int32, device=gpu)  # 9 >= seq
    rp = torch.zeros(3, dtype=torch.int32, device=gpu)
    flag = torch.zeros(1, dtype=torch.int32, device=gpu)
    w = torch.ones(R, dtype=dtype, device=gpu)
    b = torch.zeros(R, dtype=dtype, device=gpu)
    kernels.append(kv, cache, w, b, 1e-5, cos, sin, seq_idx=seq, dst_pos=dst, rope_pos=rp, err_flag=flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 1
    assert bool((cache.ckv[0, 0] != 0).any())  # the valid token landed
    assert int((cache.ckv != 0).sum()) == int((cache.ckv[0, 0] != 0).sum())


# ------------------------------------------------------------------ decode
def _decode_case(gpu, dtype, fp8, lens, n_splits, min_chunk, row_seq=None, B=None, S=None, seed=0,
                 q_scale=1.0, rope_pos=None, rtol=2e-2, atol=1e-2, rank=R, balance=0):
    rows = len(lens)
    B = B or rows
    S = S or max(max(lens), 1)
    rp_ = kernels.padded_rank(rank)
    say(f"decode case dtype={dtype} fp8={fp8} rows={rows} lens={lens[:6]}... splits={n_splits} "
        f"chunk={min_chunk} rank={rank} balance={balance}")
    g = torch.Generator().manual_seed(seed)
    cdt = torch.bfloat16 if fp8 else dtype
    # latent rows of R_pad channels, zero beyond the rank (as the append writes them)
    ckv = torch.zeros(B, S, rp_, dtype=cdt)
    ckv[..., :rank] = torch.randn(B, S, rank, generator=g).to(cdt)
    kpe = (torch.randn(B, S, P, generator=g)).to(dtype)
    if fp8:
        codes, scale = lo.fp8_quantize(ckv.reshape(-1, rp_))
        cache = LatentCache(codes.view(B, S, rp_).to(gpu), kpe.to(gpu), scale.view(B, S).to(gpu), rank)
    else:
        cache = LatentCache(ckv.to(gpu), kpe.to(gpu), rank=rank)
    # the query's padding channels hold garbage the kernel must ignore
    q_abs = (torch.randn(rows, H, rp_, generator=g) * q_scale).to(dtype)
    q_pe = (torch.randn(rows, H, P, generator=g) * q_scale).to(dtype)
    rs = torch.arange(rows, dtype=torch.int32) if row_seq is None else torch.tensor(row_seq, dtype=torch.int32)
    kl = torch.tensor(lens, dtype=torch.int32)
    rp = torch.zeros(rows, dtype=torch.int32) if rope_pos is None else torch.tensor(rope_pos, dtype=torch.int32)
    cos, sin = tables(dtype, max(S, 64), gpu)
    lse = torch.full((rows, H), float("nan"), device=gpu)
    out = kernels.decode_attention(
        q_abs.to(gpu), q_pe.to(gpu), cos, sin, cache, SCALE, row_seq=rs.to(gpu), kv_len=kl.to(gpu),
        q_rope_pos=rp.to(gpu), n_splits=n_splits, min_chunk=min_chunk, balance=balance, lse_out=lse,
    )
    torch.cuda.synchronize()
    q_pe_rot = lo.rope_interleaved(q_pe, cos.cpu()[rp.long()][:, None], sin.cpu()[rp.long()][:, None])
    ref, ref_lse = lo.absorbed_attention_f64(
        q_abs[..., :rank], q_pe_rot, cache.ckv.cpu()[..., :rank], kpe, kl, rs, SCALE,
        cache.scale.cpu() if fp8 else None
    )
    close(out[..., :rank], ref, rtol, atol)
    check_lse(lse, ref_lse)
    assert bool((out[..., rank:].float() == 0).all()), "padding channels of o_lat must be 0"
    return out


@pytest.mark.parametrize("dtype,fp8", [(torch.bfloat16, False), (torch.bfloat16, True), (torch.float32, False)])
def test_decode_short_rows(gpu, dtype, fp8):
    tol = dict(rtol=1e-4, atol=1e-5) if dtype == torch.float32 else {}
    _decode_case(gpu, dtype, fp8, [1], 1, 256, **tol)
    _decode_case(gpu, dtype, fp8, [15, 64, 100, 17], 1, 256, seed=1, **tol)
    _decode_case(gpu, dtype, fp8, [130, 1, 63, 65], 4, 64, seed=2, **tol)


@pytest.mark.parametrize("rank", [1, 64, 100, 128, 173, 200, 320, 384, 449, 512, 600, 777, 1024])
@pytest.mark.parametrize("dtype,fp8", [(torch.bfloat16, False), (torch.bfloat16, True), (torch.float32, False)])
def test_decode_any_rank(gpu, dtype, fp8, rank):
    """kv_lora_rank other than 256: one split, split-KV with the merge, and
    the balanced plan; the query padding is ignored and the output padding 0.
    Ranks above 512 run the four-chunk merge, and attention on the
    channel-split MFMA kernel (bf16 model) or the VALU kernel (fp32
    models)."""
    tol = dict(rtol=1e-4, atol=1e-5) if dtype == torch.float32 else {}
    _decode_case(gpu, dtype, fp8, [1, 70, 300], 1, 256, seed=rank, rank=rank, **tol)
    _decode_case(gpu, dtype, fp8, [1000, 1, 513, 2100], 8, 64, seed=rank + 1, rank=rank, **tol)
    _decode_case(gpu, dtype, fp8, [1000, 0, 513, 2100], 16, 64, seed=rank + 2, rank=rank, balance=256, **tol)


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("rank", [576, 640, 768, 960, 1024])
def test_decode_wide_rank_long(gpu, rank, fp8):
    """Ranks above 512 on the channel-split MFMA kernel (bf16 and e4m3
    caches) at the headline's length (the four waves own 64-channel blocks
    w, w + 4, ...: spare blocks at NB = 9, 10, 15, none at 12 and 16), with
    the graph plan's splits, peaked and flat scores, against the fp64 oracle
    with the LSE."""
    lens = [4097] * 8
    n_splits, mc = kernels.plan_splits(8, 4097)
    _decode_case(gpu, torch.bfloat16, fp8, lens, n_splits, mc, seed=rank, rank=rank, q_scale=0.5)
    _decode_case(gpu, torch.bfloat16, fp8, [4097, 17, 1, 2000], 1, 64, seed=rank + 1, rank=rank, q_scale=3.0,
                 rope_pos=[3000, 7, 0, 1999])


@pytest.mark.parametrize("dtype,fp8", [(torch.bfloat16, False), (torch.bfloat16, True), (torch.float32, False)])
def test_decode_split_kv_merge(gpu, dtype, fp8):
    tol = dict(rtol=1e-4, atol=1e-5) if dtype == torch.float32 else {}
    _decode_case(gpu, dtype, fp8, [1000, 1, 513, 4096], 8, 64, seed=3, **tol)
    _decode_case(gpu, dtype, fp8, [4096, 4096], 64, 64, seed=4, **tol)
    # more splits than a wavefront's lanes: 100 for the long rows
    _decode_case(gpu, dtype, fp8, [7000, 6500, 3, 5000], 100, 64, seed=14, **tol)


def test_decode_ragged_row_mapping_and_rope(gpu):
    """Rows map to arbitrary cache rows (prefill semantics: several query rows
    per sequence with causal lengths) and rotate q_pe at their own position."""
    row_seq = [2, 2, 2, 0, 1, 1, 3, 0]
    lens = [5, 6, 7, 300, 1, 2, 2000, 301]
    _decode_case(gpu, torch.bfloat16, False, lens, 8, 64, row_seq=row_seq, B=4, S=2048, seed=5,
                 rope_pos=[0, 1, 2, 3, 0, 1, 77, 9])


def test_decode_random_ragged_batch(gpu):
    rng = np.random.default_rng(6)
    lens = [int(x) for x in rng.integers(1, 3000, 24)]
    _decode_case(gpu, torch.bfloat16, False, lens, 16, 128, seed=6)
    _decode_case(gpu, torch.bfloat16, True, lens, 16, 128, seed=7)


def test_decode_peaked_and_flat_softmax(gpu):
    _decode_case(gpu, torch.bfloat16, False, [700, 1500], 4, 64, seed=8, q_scale=4.0)
    _decode_case(gpu, torch.bfloat16, False, [700, 1500], 4, 64, seed=9, q_scale=0.01)


def test_decode_split_invariance(gpu):
    """The merged result does not depend on the split plan (within fp32 ulps
    before the final bf16 rounding, so at most 1 bf16 ulp apart)."""
    outs = [
        _decode_case(gpu, torch.bfloat16, False, [3000, 2500, 64], ns, mc, seed=10)
        for ns, mc in ((1, 64), (8, 64), (47, 64))
    ]
    for o in outs[1:]:
        assert float((o.float() - outs[0].float()).abs().max()) <= 2 ** -7 * float(outs[0].float().abs().max())


def test_decode_constant_latent_rows(gpu):
    """All cached latent rows equal -> o_lat equals that row exactly (the
    weights sum to 1 in the kernel's own arithmetic)."""
    dtype = torch.bfloat16
    B, S = 2, 777
    row = torch.randn(R).to(dtype)
    cache = LatentCache(row.expand(B, S, R).contiguous().to(gpu), torch.randn(B, S, P).to(dtype).to(gpu))
    q_abs = torch.randn(B, H, R).to(dtype).to(gpu)
    q_pe = torch.randn(B, H, P).to(dtype).to(gpu)
    cos, sin = tables(dtype, S, gpu)
    z = torch.zeros(B, dtype=torch.int32, device=gpu)
    out = kernels.decode_attention(q_abs, q_pe, cos, sin, cache, SCALE,
                                   row_seq=torch.arange(B, dtype=torch.int32, device=gpu),
                                   kv_len=torch.tensor([S, 300], dtype=torch.int32, device=gpu),
                                   q_rope_pos=z, n_splits=1)
    torch.cuda.synchronize()
    err = (out.float().cpu() - row.float()).abs().max()
    assert float(err) <= 2 ** -8 * float(row.float().abs().max())


def test_decode_headline_shape(gpu):
    """Config-2 shape: 32 rows over 4097 cached tokens, graph-style split
    plan; o_lat and the log-sum-exp against the fp64 oracle."""
    lens = [4097] * 32
    n_splits, mc = kernels.plan_splits(32, 4097)
    _decode_case(gpu, torch.bfloat16, False, lens, n_splits, mc, seed=11, q_scale=0.5)
    _decode_case(gpu, torch.bfloat16, True, lens, n_splits, mc, seed=12, q_scale=0.5)


def test_workspace_reuse_repeated_calls(gpu):
    """Back-to-back calls that reuse one partial workspace (as a replayed
    graph does) keep giving the single-pass result."""
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(13)
    B, S = 6, 3000
    cache = LatentCache(torch.randn(B, S, R, generator=g).to(dtype).to(gpu),
                        torch.randn(B, S, P, generator=g).to(dtype).to(gpu))
    cos, sin = tables(dtype, S, gpu)
    q_abs = torch.randn(B, H, R, generator=g).to(dtype).to(gpu)
    q_pe = torch.randn(B, H, P, generator=g).to(dtype).to(gpu)
    seq = torch.arange(B, dtype=torch.int32, device=gpu)
    z = torch.zeros(B, dtype=torch.int32, device=gpu)
    ws = kernels.DecodeWorkspace.allocate(B, 16, gpu)
    outs = []
    for i in range(5):
        kl = torch.tensor([S - 7 * i, 64 + i, 1, 2000, 700 + i, S], dtype=torch.int32, device=gpu)
        ref = kernels.decode_attention(q_abs, q_pe, cos, sin, cache, SCALE, row_seq=seq, kv_len=kl,
                                       q_rope_pos=z, n_splits=1)
        got = kernels.decode_attention(q_abs, q_pe, cos, sin, cache, SCALE, row_seq=seq, kv_len=kl,
                                       q_rope_pos=z, n_splits=16, min_chunk=64, workspace=ws)
        outs.append((got.float().cpu(), ref.float().cpu()))
    torch.cuda.synchronize()
    for got, ref in outs:
        assert float((got - ref).abs().max()) <= 2 ** -7 * float(ref.abs().max())


def test_dense_addressing_equals_explicit(gpu):
    """start_pos addressing (entry i -> sequence i // T at start + i % T) gives
    the same cache bits and attention outputs as the explicit arrays."""
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(14)
    B, T, S = 3, 5, 256
    start = torch.tensor([0, 17, 200], dtype=torch.int32)
    kv = (torch.randn(B * T, 320, generator=g) * 2).to(dtype).to(gpu)
    w = (1 + 0.1 * torch.randn(R, generator=g)).to(dtype).to(gpu)
    b = (0.1 * torch.randn(R, generator=g)).to(dtype).to(gpu)
    cos, sin = tables(dtype, S, gpu)
    seq = torch.arange(B, dtype=torch.int32).repeat_interleave(T)
    t = torch.arange(T, dtype=torch.int32).repeat(B)
    dst = start.repeat_interleave(T) + t
    for rope_abs in (False, True):
        rp = dst if rope_abs else t
        c1 = LatentCache.allocate(B, S, dtype, gpu)
        c2 = LatentCache.allocate(B, S, dtype, gpu)
        kernels.append(kv, c1, w, b, 1e-5, cos, sin, seq_idx=seq.to(gpu), dst_pos=dst.to(gpu), rope_pos=rp.to(gpu))
        kernels.append(kv, c2, w, b, 1e-5, cos, sin, start_pos=start.to(gpu), tokens_per_seq=T, rope_abs=rope_abs)
        torch.cuda.synchronize()
        assert torch.equal(c1.ckv.view(torch.int16), c2.ckv.view(torch.int16))
        assert torch.equal(c1.kpe.view(torch.int16), c2.kpe.view(torch.int16))
        q_abs = torch.randn(B * T, H, R, generator=g).to(dtype).to(gpu)
        q_pe = torch.randn(B * T, H, P, generator=g).to(dtype).to(gpu)
        o1 = kernels.decode_attention(q_abs, q_pe, cos, sin, c1, SCALE, row_seq=seq.to(gpu),
                                      kv_len=(dst + 1).to(gpu), q_rope_pos=rp.to(gpu), n_splits=4, min_chunk=64)
        o2 = kernels.decode_attention(q_abs, q_pe, cos, sin, c2, SCALE, start_pos=start.to(gpu), rows_per_seq=T,
                                      rope_abs=rope_abs, n_splits=4, min_chunk=64)
        torch.cuda.synchronize()
        assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))


@pytest.mark.parametrize("dtype,fp8", [(torch.bfloat16, False), (torch.bfloat16, True), (torch.float32, False)])
def test_balanced_plan_matches_oracle_and_host_chunk(gpu, dtype, fp8):
    """A balanced launch (one chunk chosen on the device from all rows'
    lengths, 256 workgroups sharing the rows' splits) matches the fp64 oracle,
    writes the chunk mla_balanced_chunk computes on the host, and merges
    through mla_merge with that chunk.  Rows: empty, one token, ragged, a
    cache row past the batch (empty) and a length past the cache (clamped)."""
    say(f"balanced plan dtype={dtype} fp8={fp8}")
    g = torch.Generator().manual_seed(21 + fp8)
    B, S = 9, 5000
    cdt = torch.bfloat16 if fp8 else dtype
    ckv = torch.randn(B, S, R, generator=g).to(cdt)
    kpe = torch.randn(B, S, P, generator=g).to(dtype)
    if fp8:
        codes, scale = lo.fp8_quantize(ckv.reshape(-1, R))
        cache = LatentCache(codes.view(B, S, R).to(gpu), kpe.to(gpu), scale.view(B, S).to(gpu))
    else:
        cache = LatentCache(ckv.to(gpu), kpe.to(gpu))
    lens = [4999, 0, 1, 700, 64, 65, 3000, 129, 2500, 5000 + 300, 40]
    seqs = [0, 1, 2, 3, 4, 5, 6, 7, 8, 3, B + 2]  # row 9 longer than the cache, row 10 past the batch
    rows = len(lens)
    q_abs = torch.randn(rows, H, R, generator=g).to(dtype)
    q_pe = torch.randn(rows, H, P, generator=g).to(dtype)
    rp = torch.zeros(rows, dtype=torch.int32)
    cos, sin = tables(dtype, S, gpu)
    seq_t, len_t = torch.tensor(seqs, dtype=torch.int32), torch.tensor(lens, dtype=torch.int32)
    # as many workgroups as the CUs hold (one per CU: a workgroup's tile ring takes the CU's LDS)
    bal, cap = kernels.balanced_splits(rows, 256, kernels.decode_blocks_per_cu(dtype, fp8, R, False, gpu))
    assert bal == 256
    ws = DecodeWorkspace.allocate(rows, cap, gpu)
    ws.plan.fill_(-7)
    out = kernels.decode_attention(q_abs.to(gpu), q_pe.to(gpu), cos, sin, cache, SCALE, row_seq=seq_t.to(gpu),
                                   kv_len=len_t.to(gpu), q_rope_pos=rp.to(gpu), n_splits=cap, min_chunk=64,
                                   workspace=ws, balance=bal)
    torch.cuda.synchronize()
    clamped = [0 if s >= B else min(L, S) for s, L in zip(seqs, lens)]
    assert int(ws.plan.item()) == kernels.balanced_chunk(clamped, cap, 64, bal)
    q_pe_rot = lo.rope_interleaved(q_pe, cos.cpu()[rp.long()][:, None], sin.cpu()[rp.long()][:, None])
    seq_ref = torch.tensor([min(s, B - 1) for s in seqs], dtype=torch.int32)
    ref, _ = lo.absorbed_attention_f64(q_abs, q_pe_rot, cache.ckv.cpu(), kpe, torch.tensor(clamped, dtype=torch.int32),
                                       seq_ref, SCALE, cache.scale.cpu() if fp8 else None)
    tol = dict(rtol=1e-4, atol=1e-5) if dtype == torch.float32 else dict(rtol=2e-2, atol=1e-2)
    close(out, ref, **tol)
    assert bool((out[1].float() == 0).all()) and bool((out[10].float() == 0).all())


def test_e4m3_decode_every_code_exact(gpu):
    """The kernels' e4m3 -> bf16 conversion, bit for bit on every finite code.
    A row whose single cached token has scale 1 gets one softmax weight of
    exactly 1, so the output is the decoded latent row itself; 256 channels
    hold the codes 0..255 (the NaN codes 0x7f and 0xff hold 0, and so does
    -0, 0x80, which the accumulation 0 + 1 x -0 returns as +0).  The prefill
    kernel is checked on the rows that attend to 1, 2, 4 or 8 identical tokens
    (equal weights, exact 1/n)."""
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    codes[0x7F] = 0
    codes[0xFF] = 0
    codes[0x80] = 0
    expect = codes.view(torch.float8_e4m3fn).to(torch.bfloat16).view(torch.int16)
    B, S = 3, 16
    cache = LatentCache(codes.repeat(B, S, 1).to(gpu), torch.zeros(B, S, P, dtype=torch.bfloat16, device=gpu),
                        torch.ones(B, S, device=gpu))
    g = torch.Generator().manual_seed(5)
    cos, sin = tables(torch.bfloat16, 64, gpu)
    q_abs = torch.randn(B, H, R, generator=g).to(torch.bfloat16).to(gpu)
    q_pe = torch.randn(B, H, P, generator=g).to(torch.bfloat16).to(gpu)
    one = torch.ones(B, dtype=torch.int32, device=gpu)
    out = kernels.decode_attention(q_abs, q_pe, cos, sin, cache, SCALE, row_seq=torch.arange(B, dtype=torch.int32, device=gpu),
                                   kv_len=one, q_rope_pos=one * 0, n_splits=1, min_chunk=64)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu().view(torch.int16), expect.expand(B, H, R))
    T = 8
    qa = torch.randn(B * T, H, R, generator=g).to(torch.bfloat16).to(gpu)
    qp = torch.randn(B * T, H, P, generator=g).to(torch.bfloat16).to(gpu)
    out = kernels.prefill_attention(qa, qp, cos, sin, cache, SCALE, start_pos=one * 0, rows_per_seq=T)
    torch.cuda.synchronize()
    rows = [b * T + i for b in range(B) for i in (0, 1, 3, 7)]
    assert torch.equal(out.cpu()[rows].view(torch.int16), expect.expand(len(rows), H, R))


def test_decode_blocks_per_cu(gpu):
    """Workgroups per CU the split plans target: one for every cache type and
    rank (a decode workgroup's tile ring takes the CU's LDS), the fused-append
    instance included, and one for fp32."""
    for rank in (64, 128, 200, 256, 320, 512):
        for fused in (False, True):
            assert kernels.decode_blocks_per_cu(torch.bfloat16, False, rank, fused, gpu) == 1
            assert kernels.decode_blocks_per_cu(torch.bfloat16, True, rank, fused, gpu) == 1
        assert kernels.decode_blocks_per_cu(torch.float32, False, rank, False, gpu) == 1
    lib = _abi.lib()
    assert lib.mla_decode_blocks_per_cu(_abi.DTYPE_F32, _abi.DTYPE_F32, 256, 1) == -2  # no fused fp32 kernel


def test_balanced_plan_follows_lengths_in_graph_replays(gpu):
    """The plan is computed in the launch, so a captured graph replayed with
    new lengths re-balances: each replay equals an eager fixed-plan call on the
    same lengths (decode with the split merge fused into W_uv, as MLA runs it)."""
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(23)
    B, S, Dv = 24, 6000, 128
    cache = LatentCache(torch.randn(B, S, R, generator=g).to(dtype).to(gpu),
                        torch.randn(B, S, P, generator=g).to(dtype).to(gpu))
    cos, sin = tables(dtype, S, gpu)
    q_abs = torch.randn(B, H, R, generator=g).to(dtype).to(gpu)
    q_pe = torch.randn(B, H, P, generator=g).to(dtype).to(gpu)
    w_uv = (0.05 * torch.randn(H, Dv, R, generator=g)).to(dtype).to(gpu)
    sp = torch.zeros(B, dtype=torch.int32, device=gpu)
    bal, cap = kernels.balanced_splits(B, 256)
    ws = DecodeWorkspace.allocate(B, cap, gpu)
    o_lat = torch.empty(B, H, R, dtype=dtype, device=gpu)
    y = torch.empty(B, H, Dv, dtype=dtype, device=gpu)

    def step():
        kernels.decode_attention(q_abs, q_pe, cos, sin, cache, SCALE, start_pos=sp, n_splits=cap, min_chunk=64,
                                 out=o_lat, workspace=ws, merge=False, balance=bal)
        kernels.merge_project(o_lat, w_uv, y, cache, n_splits=cap, min_chunk=64, workspace=ws, start_pos=sp,
                              balanced=True)

    def fixed(lengths_sp):
        ns, mc = kernels.plan_splits(B, S)
        w2 = DecodeWorkspace.allocate(B, ns, gpu)
        o2 = torch.empty(B, H, R, dtype=dtype, device=gpu)
        y2 = torch.empty(B, H, Dv, dtype=dtype, device=gpu)
        kernels.decode_attention(q_abs, q_pe, cos, sin, cache, SCALE, start_pos=lengths_sp, n_splits=ns,
                                 min_chunk=mc, out=o2, workspace=w2, merge=False)
        kernels.merge_project(o2, w_uv, y2, cache, n_splits=ns, min_chunk=mc, workspace=w2, start_pos=lengths_sp)
        return y2

    rng = np.random.default_rng(24)
    sp.copy_(torch.tensor(rng.integers(0, S, B), dtype=torch.int32))
    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for i in range(4):
        lens = rng.integers(0, S, B) if i != 2 else np.full(B, S - 1)
        if i == 3:
            lens[:20] = 5  # a few long rows among short ones
        new_sp = torch.tensor(lens, dtype=torch.int32, device=gpu)
        sp.copy_(new_sp)
        y.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        want = fixed(new_sp.clone())
        torch.cuda.synchronize()
        clamped = [min(int(v) + 1, S) for v in lens]
        assert int(ws.plan.item()) == kernels.balanced_chunk(clamped, cap, 64, bal)
        err = float((y.float() - want.float()).abs().max())
        assert err <= 2 ** -7 * float(want.float().abs().max()) + 1e-3, (i, err)
