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


@pytest.mark.parametrize("M", [1, 7, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("K", [128, 1024, 2048])
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
