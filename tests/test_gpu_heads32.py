"""GPU parity of the 32-head decode launch (each wave serves two head groups
of 16 from one stream of the cache; the xl preset's n_head = 32 and the
cudnn-compatible 32-head layout, models/swa_mla_model.py:618-640, :696-699;
attention as models/mla.py:417-487), bf16 and e4m3 caches.

Bar: identical bits to two 16-head launches on the same inputs.  The split's
sub-tiles are dealt to the waves exactly as in a 16-head launch, each head
group runs its own online softmax on the same operands and the waves are
combined in the same fixed order, so outputs, split partials, log-sum-exps
and (with the fused append) cache rows must match bit for bit; plus the fp64
oracle at the north-star tolerance and the LSE to 1e-4."""
import pytest
import torch

from attn_ref import check, check_lse
from oracle import latent_ops as lo
from swamla_amd import kernels
from swamla_amd.kernels import DecodeWorkspace, FusedAppend, LatentCache
from swamla_amd.rope import rope_tables

pytestmark = pytest.mark.gpu

R, P = 256, 64
SCALE = 192 ** -0.5


def say(*a):
    print(*a, flush=True)


def tables(S, device):
    cos, sin = rope_tables(64, S)
    return (cos.to(torch.bfloat16)[0, 0, :, :32].contiguous().to(device),
            sin.to(torch.bfloat16)[0, 0, :, :32].contiguous().to(device))


def make(gpu, B, S, seed, rank=R, fp8=False):
    g = torch.Generator(device=gpu).manual_seed(seed)
    rp = kernels.padded_rank(rank)
    cache = LatentCache.allocate(B, S, torch.bfloat16, gpu, rank=rank, fp8=fp8)
    ckv = torch.randn(B, S, rp, generator=g, device=gpu)
    ckv[..., rank:] = 0
    if fp8:
        codes, scale = lo.fp8_quantize(ckv.to(torch.bfloat16).view(B * S, rp).cpu())
        cache.ckv.copy_(codes.view(B, S, rp))
        cache.scale.copy_(scale.view(B, S))
    else:
        cache.ckv.copy_(ckv.to(torch.bfloat16))
    cache.kpe.copy_(torch.randn(B, S, P, generator=g, device=gpu).to(torch.bfloat16))
    q_abs = (0.4 * torch.randn(B, 32, rp, generator=g, device=gpu)).to(torch.bfloat16)
    q_pe = (0.4 * torch.randn(B, 32, P, generator=g, device=gpu)).to(torch.bfloat16)
    return cache, q_abs, q_pe


def clone(c):
    return LatentCache(c.ckv.clone(), c.kpe.clone(), None if c.scale is None else c.scale.clone(), c.rank)


STARTS = [0, 15, 16, 300, 1023, 2047, 3000, 4094]


@pytest.mark.parametrize("n_splits,min_chunk", [(1, 256), (8, 256), (40, 64)])
@pytest.mark.parametrize("fused", [False, True], ids=["plain", "fused"])
@pytest.mark.parametrize("merge", [True, False], ids=["merge", "partials"])
@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "e4m3"])
def test_32_heads_equal_two_16_head_launches(gpu, n_splits, min_chunk, fused, merge, fp8):
    say(f"32 heads: n_splits={n_splits} min_chunk={min_chunk} fused={fused} merge={merge} fp8={fp8}")
    B, S = len(STARTS), 4096
    cache0, q_abs, q_pe = make(gpu, B, S, 7 + n_splits, fp8=fp8)
    cos, sin = tables(S, gpu)
    sp = torch.tensor(STARTS, dtype=torch.int32, device=gpu)
    g = torch.Generator(device=gpu).manual_seed(3)
    kv = torch.randn(B, 336, generator=g, device=gpu).to(torch.bfloat16)[:, :R + P]
    ln_w = (1 + 0.1 * torch.randn(R, generator=g, device=gpu)).to(torch.bfloat16)
    ln_b = (0.1 * torch.randn(R, generator=g, device=gpu)).to(torch.bfloat16)

    def run(heads):
        cache = clone(cache0)
        outs, lses, parts = [], [], []
        for h0 in range(0, 32, heads):
            hs = slice(h0, h0 + heads)
            ws = DecodeWorkspace.allocate(B, n_splits, gpu, heads=heads) if n_splits > 1 else None
            if ws is not None:
                ws.o_part.fill_(float("nan"))
                ws.lse_part.fill_(float("nan"))
            out = torch.full((B, heads, R), float("nan"), dtype=torch.bfloat16, device=gpu)
            lse = torch.full((B, heads), float("nan"), device=gpu)
            # each launch appends the same token (the 16-head runs write it twice, the same bits)
            fa = FusedAppend(kv, ln_w, ln_b, 1e-5) if fused else None
            kernels.decode_attention(q_abs[:, hs], q_pe[:, hs], cos, sin, cache, SCALE, start_pos=sp,
                                     n_splits=n_splits, min_chunk=min_chunk, out=out, workspace=ws,
                                     merge=merge, append=fa, lse_out=lse if merge else None)
            outs.append(out)
            lses.append(lse)
            if ws is not None:
                parts.append((ws.o_part, ws.lse_part))
        torch.cuda.synchronize()
        return cache, torch.cat(outs, 1), torch.cat(lses, 1), parts

    c32, o32, l32, p32 = run(32)
    c16, o16, l16, p16 = run(16)
    assert torch.equal(c32.ckv, c16.ckv) and torch.equal(c32.kpe, c16.kpe)
    if fp8:
        assert torch.equal(c32.scale, c16.scale)
    assert torch.equal(torch.isnan(o32), torch.isnan(o16))
    assert torch.equal(torch.nan_to_num(o32).view(torch.int16), torch.nan_to_num(o16).view(torch.int16))
    if merge:
        assert torch.equal(l32, l16)
    elif p32:
        (a32, b32), = p32
        a16 = torch.cat([p[0] for p in p16], 2)
        b16 = torch.cat([p[1] for p in p16], 2)
        assert torch.equal(torch.nan_to_num(a32), torch.nan_to_num(a16))
        assert torch.equal(torch.nan_to_num(b32), torch.nan_to_num(b16))


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "e4m3"])
def test_32_heads_against_fp64_oracle(gpu, fp8):
    say(f"32 heads vs fp64 oracle, fp8={fp8}")
    B, S, rank = 3, 1500, 200
    cache, q_abs, q_pe = make(gpu, B, S, 11, rank=rank, fp8=fp8)
    cos, sin = tables(S, gpu)
    lens = [1500, 977, 64]
    sp = torch.tensor([L - 1 for L in lens], dtype=torch.int32, device=gpu)
    lse = torch.empty(B, 32, device=gpu)
    out = kernels.decode_attention(q_abs, q_pe, cos, sin, cache, SCALE, start_pos=sp, n_splits=6, min_chunk=64,
                                   lse_out=lse)
    torch.cuda.synchronize()
    # chunk-local RoPE: a one-token row is rotated at position 0 (identity)
    o64, l64 = lo.absorbed_attention_f64(q_abs.cpu()[..., :rank], q_pe.cpu(), cache.ckv.cpu()[..., :rank],
                                         cache.kpe.cpu(), lens, [0, 1, 2], SCALE,
                                         ckv_scale=cache.scale.cpu() if fp8 else None)
    check(out.cpu()[..., :rank], o64)
    assert bool((out[..., rank:] == 0).all())
    check_lse(lse, l64)


def test_32_heads_balanced_plan_and_merge_project(gpu):
    """The length-balanced plan and the fused merge + W_uv read-out at 32
    heads equal their 16-head halves bit for bit."""
    say("32 heads: balanced plan + merge_project")
    B, S = 12, 3000
    cache, q_abs, q_pe = make(gpu, B, S, 13)
    cos, sin = tables(S, gpu)
    g = torch.Generator(device=gpu).manual_seed(5)
    lens = torch.randint(1, S + 1, (B,), generator=g, device=gpu, dtype=torch.int32)
    sp = lens - 1
    w_uv = (0.05 * torch.randn(32, 128, R, generator=g, device=gpu)).to(torch.bfloat16)
    bal, cap = kernels.balanced_splits(B, 64)
    res = {}
    for heads in (32, 16):
        ys = []
        for h0 in range(0, 32, heads):
            hs = slice(h0, h0 + heads)
            ws = DecodeWorkspace.allocate(B, cap, gpu, heads=heads)
            o_lat = torch.empty(B, heads, R, dtype=torch.bfloat16, device=gpu)
            kernels.decode_attention(q_abs[:, hs], q_pe[:, hs], cos, sin, cache, SCALE, start_pos=sp, n_splits=cap,
                                     min_chunk=64, out=o_lat, workspace=ws, merge=False, balance=bal)
            y = torch.empty(B, heads, 128, dtype=torch.bfloat16, device=gpu)
            kernels.merge_project(o_lat, w_uv[hs], y, cache, n_splits=cap, min_chunk=64, workspace=ws,
                                  start_pos=sp, balanced=True)
            ys.append(y)
        torch.cuda.synchronize()
        res[heads] = torch.cat(ys, 1)
    assert torch.equal(res[32].view(torch.int16), res[16].view(torch.int16))
