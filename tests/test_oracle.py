"""Pins of the per-kernel oracle (oracle/latent_ops.py) against library
routines, exact arithmetic, closed forms and the reference restatement."""
import ctypes
import math
import random

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import latent_ops as lo
from oracle.mla_ref import MLAConfig, RefMLA, RefRoPE, enable_cache, init_weights


# ------------------------------------------------------------------ rounding
def test_f32_to_bf16_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200_000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 200_000),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 3.3895e38, 3.4e38], np.float32),
    ]).astype(np.float32)
    ours = lo.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_host_bf16_hook_matches_torch(lib):
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(100_000) * 1e3).astype(np.float32)
    hook = np.empty(x.size, np.uint16)
    lib.mla_host_f32_to_bf16(x.ctypes.data, hook.ctypes.data, x.size)
    assert np.array_equal(hook, torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))


# ---------------------------------------------------------------------- fp8
def _e4m3_sample():
    rng = np.random.default_rng(3)
    vals = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    vals = vals[np.isfinite(vals)]
    mids = (vals[:-1] + vals[1:]) / 2 if False else None
    s = np.sort(np.unique(vals))
    mid = ((s[:-1].astype(np.float64) + s[1:]) / 2).astype(np.float32)
    near = np.concatenate([np.nextafter(mid, np.inf), np.nextafter(mid, -np.inf), mid])
    rand = rng.uniform(-470, 470, 500_000).astype(np.float32)
    tiny = (rng.uniform(-0.03, 0.03, 200_000)).astype(np.float32)
    edge = np.array([448, 463.99997, 464, 464.00003, 480, 1e9, np.inf, -np.inf, np.nan, 0.0, -0.0,
                     2.0 ** -10, 2.0 ** -9, 1.5 * 2.0 ** -9, 2.0 ** -7 * 0.999], np.float32)
    return np.concatenate([s, near, rand, tiny, edge]).astype(np.float32)


def test_e4m3_encoder_matches_torch(lib):
    x = _e4m3_sample()
    hook = np.empty(x.size, np.uint8)
    lib.mla_host_f32_to_e4m3(x.ctypes.data, hook.ctypes.data, x.size)
    ref = lo.f32_to_e4m3_codes(x)
    nan_ref = (ref & 0x7F) == 0x7F
    assert np.array_equal(nan_ref, (hook & 0x7F) == 0x7F)
    assert np.array_equal(hook[~nan_ref], ref[~nan_ref])


def test_e4m3_decoders_match_torch(lib):
    codes = np.arange(256, dtype=np.uint8)
    f = np.empty(256, np.float32)
    lib.mla_host_e4m3_to_f32(codes.ctypes.data, f.ctypes.data, 256)
    ref = lo.e4m3_codes_to_f32(codes)
    finite = np.isfinite(ref)
    assert np.array_equal(f[finite], ref[finite]) and np.all(np.isnan(f[~finite]))
    words = codes.reshape(-1, 4).copy().view(np.uint32).ravel()
    b = np.empty(256, np.uint16)
    lib.mla_host_e4m3x4_to_bf16(words.ctypes.data, b.ctypes.data, words.size)
    as_f = lo.bf16_bits_to_f32(b)
    assert np.array_equal(as_f[finite], ref[finite])


# ---------------------------------------------------------------- LayerNorm
LN_RANKS = [1, 5, 16, 64, 100, 128, 173, 192, 200, 256, 300, 320, 384, 449, 512, 600, 777, 896, 1000, 1024]


def _ln_rows(kind: str, M: int, N: int, g: torch.Generator) -> torch.Tensor:
    z = torch.randn(M, N, generator=g)
    if kind == "normal":
        return z
    if kind == "scaled":  # per-row scale over e^[-6, 6]
        return z * torch.exp(2 * torch.randn(M, 1, generator=g))
    if kind == "offset":  # large common offset: catastrophic-cancellation regime
        return z + 30 * torch.randn(M, 1, generator=g)
    if kind == "narrow":  # tiny spread around 1
        return z * 1e-3 + 1.0
    if kind == "heavy":  # heavy tails
        return z ** 3
    raise ValueError(kind)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rank", LN_RANKS)
def test_aten_layernorm_bit_exact_vs_torch(dtype, rank):
    """The oracle's LayerNorm (oracle/aten_layernorm.c) against the library
    routine the reference calls (torch.nn.functional.layer_norm on CPU,
    models/mla.py:107, :409): every output bit, plus torch's own per-row
    mean and rstd, over row families from narrow to heavy-tailed, with unit
    and random affine parameters."""
    g = torch.Generator().manual_seed(1000 + rank)
    for kind in ("normal", "scaled", "offset", "narrow", "heavy"):
        x = _ln_rows(kind, 1500, rank, g).to(dtype)
        for affine in (False, True):
            if affine:
                w = (1 + 0.5 * torch.randn(rank, generator=g)).to(dtype)
                b = (0.3 * torch.randn(rank, generator=g)).to(dtype)
            else:
                w, b = torch.ones(rank, dtype=dtype), torch.zeros(rank, dtype=dtype)
            y, mean, rstd = lo.layernorm_aten(x, w, b, 1e-5)
            ref = F.layer_norm(x, (rank,), w, b, 1e-5)
            assert torch.equal(y.view(torch.uint8), ref.view(torch.uint8)), f"{kind} affine={affine}: output bits"
            # fp32 parameters make torch return its fp32 statistics for bf16 input
            _, m_t, r_t = torch.native_layer_norm(x, [rank], w.float() if dtype == torch.bfloat16 else w,
                                                  b.float() if dtype == torch.bfloat16 else b, 1e-5)
            assert torch.equal(mean, m_t.view(-1)) and torch.equal(rstd, r_t.view(-1)), f"{kind}: statistics"


@pytest.mark.parametrize("variant,dtype,rank", [
    (1, torch.bfloat16, 256),   # Welford m1 update without its fused multiply-add
    (2, torch.bfloat16, 512),   # stack merge m1 update fused (two chunks)
    (2, torch.float32, 384),    # ... and for fp32 rows (three chunks at rank 384)
    (2, torch.float32, 840),    # ... seven chunks (the last short): a three-level stack
    (2, torch.bfloat16, 800),   # ... four chunks of bf16 vectors (the last short)
    (4, torch.bfloat16, 256),   # lane merge m2 associated the other way
    (8, torch.bfloat16, 256),   # affine without fused multiply-adds
    (8, torch.float32, 256),
])
def test_aten_layernorm_planted_mistakes_are_caught(variant, dtype, rank):
    """Each single-site change of the statement disagrees with torch on these
    rows, so the bit-exact comparison above pins every site it touches."""
    g = torch.Generator().manual_seed(77)
    x = _ln_rows("scaled", 4000, rank, g).to(dtype)
    w = (1 + 0.5 * torch.randn(rank, generator=g)).to(dtype)
    b = (0.3 * torch.randn(rank, generator=g)).to(dtype)
    ref = F.layer_norm(x, (rank,), w, b, 1e-5)
    good = lo.layernorm_aten(x, w, b, 1e-5)[0]
    bad = lo.layernorm_aten(x, w, b, 1e-5, variant=variant)[0]
    assert torch.equal(good.view(torch.uint8), ref.view(torch.uint8))
    assert not torch.equal(bad.view(torch.uint8), ref.view(torch.uint8))


@pytest.mark.parametrize("rank", [1, 64, 173, 256, 512])
def test_aten_layernorm_near_exact_mathematics(rank):
    """Sanity against the mathematics: within 1 bf16 ulp of the fp64
    LayerNorm, and a normalised row (unit affine) has mean ~0 and variance
    ~1 in fp64.  A single channel normalises to the rounding error of
    rstd * x (rstd = eps^-1/2), as in torch: tiny, not exactly 0."""
    g = torch.Generator().manual_seed(9)
    x = (torch.randn(2000, rank, generator=g) * 3 + 0.5).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(rank, generator=g)).to(torch.bfloat16)
    b = (0.1 * torch.randn(rank, generator=g)).to(torch.bfloat16)
    y1 = lo.layernorm_aten(x, torch.ones(rank, dtype=torch.bfloat16), torch.zeros(rank, dtype=torch.bfloat16),
                           1e-5)[0].double()
    if rank == 1:
        assert float(y1.abs().max()) <= 2.0 ** -10
        return
    y = lo.layernorm_aten(x, w, b, 1e-5)[0]
    exact = F.layer_norm(x.double(), (rank,), w.double(), b.double(), float(np.float32(1e-5)))
    ulp = torch.abs(exact).clamp(min=2.0 ** -10).log2().floor().exp2() * 2.0 ** -7
    assert bool(((y.double() - exact).abs() <= ulp * 1.0001).all())
    assert float(y1.mean(dim=1).abs().max()) < 2e-2
    assert float((y1.var(dim=1, unbiased=False) - 1).abs().max()) < 2e-2


# --------------------------------------------------------------------- RoPE
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_statement_matches_reference_rope(dtype):
    rope = RefRoPE(64, 128).to(dtype)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 3, 40, 64, generator=g).to(dtype)
    ref = rope(x)
    cos = rope.cos_cached[0, 0, :40, :32]
    sin = rope.sin_cached[0, 0, :40, :32]
    ours = lo.rope_interleaved(x, cos, sin)
    assert torch.equal(ours, ref)
    # position 0 is the identity
    assert torch.equal(ours[:, :, 0], x[:, :, 0])


def test_rope_preserves_pair_norms_fp64():
    rope = RefRoPE(64, 256).double()
    x = torch.randn(1, 1, 256, 64, dtype=torch.float64)
    y = rope(x)
    nx = x.view(1, 1, 256, 32, 2).pow(2).sum(-1)
    ny = y.view(1, 1, 256, 32, 2).pow(2).sum(-1)
    # the table itself is fp32 (cos^2 + sin^2 = 1 to ~2^-23), so the rotation
    # preserves pair norms to that accuracy, and not better
    assert torch.allclose(nx, ny, rtol=5e-7, atol=0)


def test_rope_growth_equals_a_longer_table():
    """Growth (positional_encoding.py:44-46, :64-86) on the CPU rebuilds the
    table with the same ops, so a grown table equals one built at the longer
    length bit for bit, its entries are cos / sin of t * base^(-2i/dim)
    (fp64 closed form, to fp32 accuracy), and it stays fp32 whatever the
    module dtype was."""
    rope = RefRoPE(64, 16).to(torch.bfloat16)
    x = torch.randn(1, 2, 40, 64).to(torch.bfloat16)
    y = rope(x)
    assert rope.max_seq_len == 40 and rope.cos_cached.dtype == torch.float32
    fresh = RefRoPE(64, 40)
    assert torch.equal(rope.cos_cached, fresh.cos_cached) and torch.equal(rope.sin_cached, fresh.sin_cached)
    t = torch.arange(40, dtype=torch.float64)[:, None]
    ang = t * 10000.0 ** (-torch.arange(0, 64, 2, dtype=torch.float64) / 64)
    assert torch.allclose(rope.cos_cached[0, 0, :, :32].double(), ang.cos(), atol=4e-6, rtol=0)
    assert torch.allclose(rope.sin_cached[0, 0, :, :32].double(), ang.sin(), atol=4e-6, rtol=0)
    # the rotation after growth is bf16 x fp32, so its result is fp32
    assert y.dtype == torch.float32


def test_ref_module_growth_fp32_and_bf16():
    """No-cache calls longer than max_seq_len: an fp32 module's output equals
    that of a module built with a longer table (growth changes nothing else);
    a bf16 module's grown fp32 rotation meets bf16 values in SDPA, which
    raises (mla.py:555-601)."""
    g = torch.Generator().manual_seed(21)
    x = torch.randn(1, 40, 128, generator=g)
    outs = []
    for L in (16, 64):
        m = RefMLA(MLAConfig(n_embd=128, max_batch_size=1, max_seq_len=L))
        init_weights(m, 22)
        m.eval()
        with torch.no_grad():
            outs.append(m(x, 0))
    assert torch.equal(outs[0], outs[1])
    m = RefMLA(MLAConfig(n_embd=128, max_batch_size=1, max_seq_len=16))
    init_weights(m, 22)
    m.eval().to(torch.bfloat16)
    with torch.no_grad(), pytest.raises(RuntimeError):
        m(x.to(torch.bfloat16), 0)


# ---------------------------------------------------------------- attention
def _unabsorbed_f64(q_nope, q_pe, c, kpe, w_uk, w_uv, scale):
    """mla.py:427-437 + SDPA in fp64 for one row: q [H, .], c [L, R]."""
    k_nope = torch.einsum("tc,hdc->thd", c, w_uk)  # [L, H, Dn]
    v = torch.einsum("tc,hdc->thd", c, w_uv)
    s = (torch.einsum("hd,thd->ht", q_nope, k_nope) + q_pe @ kpe.T) * scale
    return torch.einsum("ht,thd->hd", torch.softmax(s, -1), v)


def test_absorbed_equals_unabsorbed_fp64():
    g = torch.Generator().manual_seed(7)
    Hh, R, P, Dn, L = 16, 256, 64, 128, 37
    q_nope = torch.randn(Hh, Dn, generator=g, dtype=torch.float64)
    q_pe = torch.randn(Hh, P, generator=g, dtype=torch.float64)
    c = torch.randn(1, L, R, generator=g, dtype=torch.float64)
    kpe = torch.randn(1, L, P, generator=g, dtype=torch.float64)
    w_uk = torch.randn(Hh, Dn, R, generator=g, dtype=torch.float64) * 0.05
    w_uv = torch.randn(Hh, 128, R, generator=g, dtype=torch.float64) * 0.05
    scale = 192 ** -0.5
    q_abs = torch.einsum("hd,hdc->hc", q_nope, w_uk)
    o_lat, _ = lo.absorbed_attention_f64(q_abs[None], q_pe[None], c, kpe, [L], [0], scale)
    o = torch.einsum("hc,hdc->hd", o_lat[0], w_uv)
    ref = _unabsorbed_f64(q_nope, q_pe, c[0], kpe[0], w_uk, w_uv, scale)
    assert torch.allclose(o, ref, rtol=1e-12, atol=1e-12)


def test_attention_closed_forms():
    g = torch.Generator().manual_seed(8)
    c = torch.randn(1, 10, 256, generator=g, dtype=torch.float64)
    kpe = torch.randn(1, 10, 64, generator=g, dtype=torch.float64)
    q = torch.randn(1, 16, 256, generator=g, dtype=torch.float64)
    qp = torch.randn(1, 16, 64, generator=g, dtype=torch.float64)
    # one cached token: o = c_0
    o, lse = lo.absorbed_attention_f64(q, qp, c, kpe, [1], [0], 0.1)
    assert torch.allclose(o[0], c[0, :1].expand(16, -1))
    # zero query: uniform weights, o = mean of c, lse = log L
    o, lse = lo.absorbed_attention_f64(torch.zeros_like(q), torch.zeros_like(qp), c, kpe, [10], [0], 0.1)
    assert torch.allclose(o[0], c[0].mean(0).expand(16, -1))
    assert torch.allclose(lse, torch.full_like(lse, math.log(10)))


def test_merge_of_splits_equals_single_pass():
    g = torch.Generator().manual_seed(9)
    L = 300
    c = torch.randn(1, L, 256, generator=g, dtype=torch.float64)
    kpe = torch.randn(1, L, 64, generator=g, dtype=torch.float64)
    q = torch.randn(1, 16, 256, generator=g, dtype=torch.float64)
    qp = torch.randn(1, 16, 64, generator=g, dtype=torch.float64)
    full, lse_full = lo.absorbed_attention_f64(q, qp, c, kpe, [L], [0], 0.07)
    parts, lses = [], []
    for a, b in [(0, 64), (64, 128), (128, 300)]:
        o, l_ = lo.absorbed_attention_f64(q, qp, c[:, a:b], kpe[:, a:b], [b - a], [0], 0.07)
        parts.append(o)
        lses.append(l_)
    o, lse = lo.merge_partials_f64(torch.stack(parts), torch.stack(lses))
    assert torch.allclose(o, full, rtol=1e-12, atol=1e-12)
    assert torch.allclose(lse, lse_full, rtol=1e-12, atol=1e-12)
    # permutation invariance and single-split identity
    o2, _ = lo.merge_partials_f64(torch.stack(parts[::-1]), torch.stack(lses[::-1]))
    assert torch.allclose(o2, o, rtol=1e-12, atol=1e-12)
    o1, l1 = lo.merge_partials_f64(torch.stack(parts[:1]), torch.stack(lses[:1]))
    assert torch.equal(o1, parts[0]) and torch.allclose(l1, lses[0])


def test_split_plan_matches_library(lib):
    rng = random.Random(10)
    for _ in range(5000):
        L = rng.randint(-2, 200_000)
        ns = rng.randint(1, 300)
        mc = rng.randint(1, 4096)
        ours = lo.split_count(L, ns, mc)
        assert lib.mla_split_count(L, ns, mc) == ours
        if L > 0:
            ch = lo.split_chunk(L, ns, mc)
            assert 1 <= ours <= ns and (ours - 1) * ch < L <= ours * ch and ch % 16 == 0


# --------------------------------------------------------- whole-path oracle
def test_fp8_emulation_error_bound():
    """e4m3 per-token quantisation keeps every element within half a code
    step: |y - deq| <= 2^-4 * |y| (normal range) or scale * 2^-10 (subnormal)."""
    g = torch.Generator().manual_seed(11)
    y = (torch.randn(64, 256, generator=g) * 2).to(torch.bfloat16)
    codes, scale = lo.fp8_quantize(y)
    deq = lo.fp8_dequantize(codes, scale)
    err = (deq - y.float()).abs()
    bound = torch.maximum(y.float().abs() * 2.0 ** -4, scale[:, None] * 2.0 ** -10)
    assert bool((err <= bound * (1 + 1e-6)).all())
    assert int(codes.max()) <= 0xFE and not bool(((codes & 0x7F) == 0x7F).any())


def test_fp8_amax_encodes_to_e4m3_max():
    """The saturation constant is e4m3fn's 448: each token's largest element
    encodes to code 0x7E (+448) or 0xFE (-448) and dequantises back to exactly
    that element up to fp32 rounding (an e4m3fnuz-style 240 divisor codes it
    0x77 / 0xF7)."""
    g = torch.Generator().manual_seed(12)
    y = (torch.randn(512, 256, generator=g) * torch.exp(torch.randn(512, 1, generator=g))).to(torch.bfloat16)
    codes, scale = lo.fp8_quantize(y)
    yf = y.float()
    idx = yf.abs().argmax(dim=1)
    top = codes[torch.arange(512), idx]
    sign = yf[torch.arange(512), idx] < 0
    assert torch.equal(top, torch.where(sign, 0xFE, 0x7E).to(torch.uint8))
    deq = lo.fp8_dequantize(codes, scale)
    # 448 * fl(amax / 448) is amax up to the two fp32 roundings
    assert torch.allclose(deq[torch.arange(512), idx], yf[torch.arange(512), idx], rtol=2.0 ** -22, atol=0)
    # the same check rejects the fnuz-style divisor
    bad_scale = yf.abs().amax(dim=1) / 240.0
    bad = (yf / bad_scale[:, None]).to(torch.float8_e4m3fn).view(torch.uint8)
    assert not torch.equal(bad[torch.arange(512), idx], top)


def test_ref_module_decode_equals_recompute():
    """The restatement's cache path against its no-cache path (fp32).
    With the rope projections zeroed (q_pe = k_pe = 0, so RoPE positions play
    no part), a 5-token prefill followed by a cached one-token decode gives
    the last position of one causal 6-token forward without a cache.  With
    RoPE active, the cached c_kv rows match those of a 6-token prefill (to
    the projections' rounding), k_pe rows 0..4 too, and row 5 is the
    un-rotated k_pe: the decode call rotates
    its token by position 0 (chunk-local positions, positional_encoding.py:
    49-50)."""
    cfg = MLAConfig(n_embd=128, max_batch_size=1, max_seq_len=16)
    g = torch.Generator().manual_seed(13)
    x = torch.randn(1, 6, 128, generator=g)

    def module(rope_zero):
        m = RefMLA(cfg)
        init_weights(m, 12)
        m.eval()
        if rope_zero:
            with torch.no_grad():
                m.wq.weight.view(16, 192, 128)[:, 128:] = 0
                m.wkv_a.weight[256:] = 0
        return m

    cached, plain = module(True), module(True)
    enable_cache(cached)
    with torch.no_grad():
        cached(x[:, :5], 0)
        dec = cached(x[:, 5:6], 5)
        full = plain(x, 0)  # no cache: causal SDPA over the 6 tokens
    assert dec.shape == (1, 1, 128)
    err = (dec - full[:, 5:6]).abs().max().item()
    assert err <= 1e-6 * max(1.0, full.abs().max().item()), err
    # the same comparison with a one-position mismatch must fail
    assert (dec - full[:, 4:5]).abs().max().item() > 1e-3

    a, b = module(False), module(False)
    enable_cache(a)
    enable_cache(b)
    with torch.no_grad():
        a(x[:, :5], 0)
        a(x[:, 5:6], 5)
        b(x, 0)
        _, _, _, k_pe_last = b.project(x[:, 5:6])
    # (the projections over 5 + 1 rows and over 6 rows may round differently)
    assert (a.kv_cache[:, :6] - b.kv_cache[:, :6]).abs().max().item() <= 1e-5
    assert (a.pe_cache[:, :5] - b.pe_cache[:, :5]).abs().max().item() <= 1e-5
    assert torch.equal(a.pe_cache[0, 5], k_pe_last.reshape(-1))
    assert (a.pe_cache[0, 5] - b.pe_cache[0, 5]).abs().max().item() > 1e-2
