"""GPU parity of mla_linear (the decode step's batched small-row products)
against an fp32 product of the same bf16 operands.

Bar: the kernel accumulates in fp32 in its own order and rounds once, so each
output is within one bf16 ulp of the fp32 reference rounded to bf16 (plus a
tiny absolute slack for results that cancel to near zero).
"""
import pytest
import torch

from swamla_amd import kernels

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def ref_linear(x, w, bias=None):
    """fp32 product on the CPU of the bf16 operands: [b, M, K] x [b, N, K]."""
    y = torch.matmul(x.float().cpu(), w.float().cpu().transpose(-1, -2))
    if bias is not None:
        y = y + bias.float().cpu().unsqueeze(-2)
    return y


def assert_within_ulp(out, ref):
    out = out.float().cpu()
    ulp = torch.finfo(torch.bfloat16).eps * ref.abs().clamp_min(2.0 ** -100)
    err = (out - ref).abs()
    bad = err > ulp + 1e-6 * ref.abs().max()
    assert not bool(bad.any()), f"{int(bad.sum())} / {bad.numel()} beyond 1 ulp; max err {float(err.max()):.3e}"


@pytest.mark.parametrize("M", [1, 7, 16, 17, 32, 33, 64, 80, 128])
@pytest.mark.parametrize("K", [128, 1024, 1152, 1536, 2048])
def test_linear_shapes(gpu, M, K):
    say(f"linear M={M} K={K}")
    g = torch.Generator().manual_seed(M * 7 + K)
    N = 48
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    out = kernels.linear(x.to(gpu), w.to(gpu))
    torch.cuda.synchronize()
    assert out.shape == (M, N)
    assert_within_ulp(out, ref_linear(x, w))


def test_linear_bias_and_stacked_projection(gpu):
    """The decode step's first product: x[32, 1024] against wq and wkv_a stacked."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(32, 1024, generator=g).to(torch.bfloat16)
    w = (torch.randn(3072 + 320, 1024, generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(3072 + 320, generator=g) * 0.1).to(torch.bfloat16)
    out = kernels.linear(x.to(gpu), w.to(gpu), bias=b.to(gpu))
    torch.cuda.synchronize()
    assert_within_ulp(out, ref_linear(x, w, b))


def test_linear_head_batched_strided_views(gpu):
    """Absorption layout: x = q[:, :, :128] of a [n, 3392] buffer viewed per
    head, w = W_uk^T [H, 256, 128], out = q_abs [n, H, 256] viewed per head;
    then the W_uv read-out straight from a wkv_b-shaped weight view."""
    g = torch.Generator().manual_seed(2)
    n, H = 32, 16
    y = torch.randn(n, 3392, generator=g).to(torch.bfloat16).to(gpu)
    q = y[:, :3072].view(n, H, 192)
    w_uk_t = (torch.randn(H, 256, 128, generator=g) * 0.05).to(torch.bfloat16).to(gpu)
    q_abs = torch.full((n, H, 256), float("nan"), dtype=torch.bfloat16, device=gpu)
    kernels.linear(q[:, :, :128].transpose(0, 1), w_uk_t, out=q_abs.transpose(0, 1))
    wkv_b = (torch.randn(H * 256, 256, generator=g) * 0.05).to(torch.bfloat16).to(gpu)
    w_uv = wkv_b.view(H, 256, 256)[:, 128:, :]
    o = torch.full((n, H * 128), float("nan"), dtype=torch.bfloat16, device=gpu)
    kernels.linear(q_abs.transpose(0, 1), w_uv, out=o.view(n, H, 128).transpose(0, 1))
    torch.cuda.synchronize()
    ref_qabs = ref_linear(q[:, :, :128].transpose(0, 1).cpu(), w_uk_t.cpu())  # [H, n, 256]
    assert_within_ulp(q_abs.transpose(0, 1), ref_qabs)
    ref_o = ref_linear(q_abs.transpose(0, 1).cpu(), w_uv.cpu())  # [H, n, 128]
    assert_within_ulp(o.view(n, H, 128).transpose(0, 1), ref_o)


def test_linear_rows_beyond_m_untouched(gpu):
    """Rows past M in the output buffer are never written."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 256, generator=g).to(torch.bfloat16).to(gpu)
    w = torch.randn(32, 256, generator=g).to(torch.bfloat16).to(gpu)
    buf = torch.full((8, 32), 7.0, dtype=torch.bfloat16, device=gpu)
    kernels.linear(x, w, out=buf[:5])
    torch.cuda.synchronize()
    assert bool((buf[5:] == 7.0).all())
    assert_within_ulp(buf[:5], ref_linear(x.cpu(), w.cpu()))


@pytest.mark.parametrize("n_splits,min_chunk,R", [(1, 64, 256), (8, 64, 256), (47, 64, 256), (100, 64, 256),
                                                  (8, 64, 320), (47, 64, 512)])
def test_merge_project_equals_merge_then_product(gpu, n_splits, min_chunk, R):
    """mla_merge_project == mla_merge followed by the W_uv product, on ragged
    rows (empty, single-split and multi-split rows in one call); up to 100
    splits per row (more than the 32 lanes that hold a row's statistics) and
    latent widths past one 256-channel chunk."""
    from swamla_amd.kernels import DecodeWorkspace, LatentCache
    from swamla_amd.rope import rope_tables

    say(f"merge_project n_splits={n_splits} R={R}")
    g = torch.Generator().manual_seed(20 + n_splits + R)
    B, H = 5, 16
    S = 7000 if n_splits > 64 else 3000
    dt = torch.bfloat16
    cache = LatentCache(torch.randn(B, S, R, generator=g).to(dt).to(gpu),
                        torch.randn(B, S, 64, generator=g).to(dt).to(gpu), rank=R)
    cos, sin = rope_tables(64, S)
    cos = cos.to(dt)[0, 0, :, :32].contiguous().to(gpu)
    sin = sin.to(dt)[0, 0, :, :32].contiguous().to(gpu)
    rows = 11
    row_seq = torch.tensor([0, 1, 2, 3, 4, 0, 1, 2, 3, 4, 1], dtype=torch.int32, device=gpu)
    kv_len = torch.tensor([S - 1, 1, 64, 65, 0, 777, S, 1500, 130, 17, 2048], dtype=torch.int32, device=gpu)
    qrp = torch.zeros(rows, dtype=torch.int32, device=gpu)
    q_abs = (torch.randn(rows, H, R, generator=g) * 0.3).to(dt).to(gpu)
    q_pe = (torch.randn(rows, H, 64, generator=g) * 0.3).to(dt).to(gpu)
    wkv_b = (torch.randn(H * 256, R, generator=g) * 0.05).to(dt).to(gpu)
    w_uv = wkv_b.view(H, 256, R)[:, 128:, :]
    ws = DecodeWorkspace.allocate(rows, n_splits, gpu, rank=R) if n_splits > 1 else None
    o_lat = torch.empty(rows, H, R, dtype=dt, device=gpu)
    kernels.decode_attention(q_abs, q_pe, cos, sin, cache, 0.0721, row_seq=row_seq, kv_len=kv_len,
                             q_rope_pos=qrp, n_splits=n_splits, min_chunk=min_chunk, out=o_lat,
                             workspace=ws, merge=False)
    got = torch.full((rows, H * 128), float("nan"), dtype=dt, device=gpu)
    kernels.merge_project(o_lat, w_uv, got.view(rows, H, 128), cache, n_splits=n_splits, min_chunk=min_chunk,
                          workspace=ws, row_seq=row_seq, kv_len=kv_len)
    # reference: the same decode with its own merge, then the per-head product
    o_ref = kernels.decode_attention(q_abs, q_pe, cos, sin, cache, 0.0721, row_seq=row_seq, kv_len=kv_len,
                                     q_rope_pos=qrp, n_splits=n_splits, min_chunk=min_chunk)
    torch.cuda.synchronize()
    ref = ref_linear(o_ref.transpose(0, 1).cpu(), w_uv.cpu())  # [H, rows, 128], fp32
    got_h = got.view(rows, H, 128).transpose(0, 1).float().cpu()
    assert not bool(torch.isnan(got_h).any())
    # The output is rounded to bf16 (up to 2^-8 relative, ~2^-10 on average);
    # merged rows are rounded to bf16 before the product in both paths, and the
    # two merges may differ by one bf16 ulp in a few channels.
    err = (got_h - ref).abs()
    assert float(err.max()) <= 2e-2 * float(ref.abs().max()), float(err.max())
    assert float(err.mean()) <= 3e-3 * float(ref.abs().mean()), float(err.mean())


def test_pack_weight_layout(gpu):
    """Packed element (n, k) sits at (((n/8)*(K/64) + k/64)*8 + (k%64)/8)*64 + (n%8)*8 + k%8."""
    N, K = 24, 192
    w = torch.arange(N * K, dtype=torch.float32).view(N, K)  # distinct values, exact in bf16 up to 256
    w = (w % 251).to(torch.bfloat16)
    buf = torch.zeros(N, K + 64, dtype=torch.bfloat16)
    buf[:, :K] = w
    wp = kernels.pack_weight(buf.to(gpu)[:, :K])
    torch.cuda.synchronize()
    n = torch.arange(N).view(N, 1)
    k = torch.arange(K).view(1, K)
    idx = (((n // 8) * (K // 64) + k // 64) * 8 + (k % 64) // 8) * 64 + (n % 8) * 8 + k % 8
    expect = torch.empty(N * K, dtype=torch.bfloat16)
    expect[idx.reshape(-1)] = w.reshape(-1)
    assert torch.equal(wp.data.cpu(), expect)


@pytest.mark.parametrize("M", [1, 7, 16, 17, 32, 33, 64, 65, 100, 128])
@pytest.mark.parametrize("N,K", [(5440, 1024), (1024, 2048), (1536, 1536), (40, 512), (8, 1024), (2056, 2048)])
def test_linear_packed_shapes(gpu, M, N, K):
    say(f"linear_packed M={M} N={N} K={K}")
    g = torch.Generator().manual_seed(M * 13 + N + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    b = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16)
    wp = kernels.pack_weight(w.to(gpu))
    out = kernels.linear_packed(x.to(gpu), wp, bias=b.to(gpu))
    torch.cuda.synchronize()
    assert out.shape == (M, N)
    assert_within_ulp(out, ref_linear(x, w, b))


def test_linear_packed_strided_rows_and_untouched_tail(gpu):
    """x and out as row-strided views (the decode step's wkv_a / wo buffers);
    rows past M and columns past N of the output buffer are never written."""
    g = torch.Generator().manual_seed(5)
    M, N, K = 32, 1024, 2048
    xb = torch.randn(M, K + 128, generator=g).to(torch.bfloat16).to(gpu)
    x = xb[:, 64:64 + K]
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    wp = kernels.pack_weight(w.to(gpu))
    buf = torch.full((M + 3, N + 40), 7.0, dtype=torch.bfloat16, device=gpu)
    kernels.linear_packed(x, wp, out=buf[:M, 8:8 + N])
    torch.cuda.synchronize()
    assert bool((buf[M:] == 7.0).all()) and bool((buf[:, :8] == 7.0).all()) and bool((buf[:, 8 + N:] == 7.0).all())
    assert_within_ulp(buf[:M, 8:8 + N], ref_linear(x.cpu(), w))


def test_linear_packed_equals_in_graph_replays(gpu):
    """Captured in a HIP graph and replayed with eager work in between, every
    replay equals the eager result bit for bit."""
    g = torch.Generator().manual_seed(6)
    x = torch.randn(32, 1024, generator=g).to(torch.bfloat16).to(gpu)
    wp = kernels.pack_weight((torch.randn(5440, 1024, generator=g) * 0.05).to(torch.bfloat16).to(gpu))
    eager = kernels.linear_packed(x, wp)
    out = torch.empty_like(eager)
    s = torch.cuda.Stream(gpu)
    s.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(s):
        kernels.linear_packed(x, wp, out=out)
    torch.cuda.current_stream(gpu).wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kernels.linear_packed(x, wp, out=out)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        _ = (x.float() * 2).sum()  # unrelated eager work between replays


@pytest.mark.parametrize("M,n_adv", [(32, 32), (128, 128), (1, 1), (100, 512)])
def test_linear_packed_advances_positions(gpu, M, n_adv):
    """The optional position advance: each entry gains exactly 1 per launch,
    eager and in graph replays, and the product's bits do not change."""
    say(f"linear_packed advance M={M} n={n_adv}")
    g = torch.Generator().manual_seed(40 + M)
    x = torch.randn(M, 2048, generator=g).to(torch.bfloat16).to(gpu)
    wp = kernels.pack_weight((torch.randn(1024, 2048, generator=g) * 0.05).to(torch.bfloat16).to(gpu))
    plain = kernels.linear_packed(x, wp)
    pos0 = torch.randint(0, 1 << 20, (n_adv,), generator=g, dtype=torch.int32)
    buf = torch.full((n_adv + 8,), -7, dtype=torch.int32, device=gpu)  # guard entries past the tensor
    pos = buf[:n_adv]
    pos.copy_(pos0.to(gpu))
    out = kernels.linear_packed(x, wp, advance=pos)
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    assert torch.equal(pos.cpu(), pos0 + 1)
    assert bool((buf[n_adv:] == -7).all())
    s = torch.cuda.Stream(gpu)
    s.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(s):
        kernels.linear_packed(x, wp, out=out, advance=pos)
    torch.cuda.current_stream(gpu).wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kernels.linear_packed(x, wp, out=out, advance=pos)
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, plain)
        assert torch.equal(pos.cpu(), pos0 + 3 + i)
        _ = (x.float() * 2).sum()  # unrelated eager work between replays
    with pytest.raises(ValueError):
        kernels.linear_packed(x, wp, advance=pos.to(torch.int64))
