"""GPU parity of mla_head_product (the prompt pass's per-head absorbed
products q_nope . W_uk and o_lat . W_uv^T, re-associating models/mla.py:427
and :433) against an fp64 product of the same bf16 operands on the CPU.

Bar: the kernel accumulates in fp32 and rounds once to nearest-even, so every
output is within one bf16 ulp of the exact product plus the fp32 summation
error bound K 2^-24 sum_k |x_k w_k| (which only matters where the terms cancel
to near zero), and all but the few whose exact value lies within that error
of a rounding boundary equal the exact product rounded to bf16 (asserted: at
least 99.5 % of them).
"""
import pytest
import torch

from swamla_amd import kernels

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def ref_head_product(x, w):
    """Exact (fp64) per-head product of the bf16 operands, [M, H, K] x
    [H, N, K], and the fp32 summation error bound of each output."""
    xd, wd = x.double().cpu(), w.double().cpu()
    ref = torch.einsum("mhk,hnk->mhn", xd, wd)
    slack = torch.einsum("mhk,hnk->mhn", xd.abs(), wd.abs()) * (x.shape[-1] * 2.0 ** -24)
    return ref, slack


def check(out, ref_slack):
    ref, slack = ref_slack
    out = out.cpu()
    exact = ref.to(torch.bfloat16)  # rounded through fp32: its rare double roundings fall in the allowance
    ulp = torch.finfo(torch.bfloat16).eps * ref.abs()
    err = (out.double() - ref).abs()
    bad = err > ulp + slack
    assert not bool(bad.any()), f"{int(bad.sum())} / {bad.numel()} beyond 1 ulp; max err {float(err.max()):.3e}"
    same = (out.view(torch.int16) == exact.view(torch.int16)).float().mean().item()
    assert same >= 0.995, f"only {same:.4f} of outputs equal the exactly rounded product"


def _operands(M, H, K, N, seed, x_cols=None):
    """x as the K leading columns of [M, H, x_cols] rows (the q_nope view of
    the wq output when x_cols = 192), w [H, N, K]."""
    g = torch.Generator().manual_seed(seed)
    xc = K if x_cols is None else x_cols
    xb = torch.randn(M, H, xc, generator=g).to(torch.bfloat16)
    w = (torch.randn(H, N, K, generator=g) * 0.06).to(torch.bfloat16)
    return xb, xb[:, :, :K], w


@pytest.mark.parametrize("M", [1, 15, 64, 65, 1000, 2000, 3001, 4099])
def test_query_absorption_shapes(gpu, M):
    """q_abs = q_nope . W_uk: x read in place from [M, 16, 192] rows, K = 128,
    N = R_pad = 256, ragged last row tile.  At 16 heads the grid has 16 blocks
    per head, so M = 2000, 3001 and 4099 give blocks two to five row tiles of
    64 whose last one is partial (down to 3 valid rows): the loader must still
    count every tile's DMAs alike."""
    say(f"head_product q-side M={M}")
    xb, x, w = _operands(M, 16, 128, 256, M, x_cols=192)
    out = kernels.head_product(xb.to(gpu)[:, :, :128], w.to(gpu))
    torch.cuda.synchronize()
    assert out.shape == (M, 16, 256)
    check(out, ref_head_product(x, w))


@pytest.mark.parametrize("M", [1, 33, 64, 777, 2100, 3000, 4097])
def test_value_readout_shapes(gpu, M):
    """o = o_lat . W_uv^T: x = o_lat [M, 16, 256], K = 256, N = 128, written
    into wo's input layout [M, 16 * 128].  M = 2100 and 3000 give blocks two
    or three row tiles with a partial last one."""
    say(f"head_product o-side M={M}")
    _, x, w = _operands(M, 16, 256, 128, 100 + M)
    out = torch.full((M, 16 * 128), float("nan"), dtype=torch.bfloat16, device=gpu)
    kernels.head_product(x.to(gpu), w.to(gpu), out=out.view(M, 16, 128))
    torch.cuda.synchronize()
    check(out.view(M, 16, 128), ref_head_product(x, w))


@pytest.mark.parametrize("K,N", [(64, 256), (128, 512), (128, 192), (192, 128), (320, 128), (448, 128),
                                 (512, 128), (64, 64), (512, 20)])
def test_other_ranks_and_head_dims(gpu, K, N):
    """Every built K (latent ranks R_pad = 64 .. 512 on the o side, 64 / 128
    nope dims on the q side) and N not a multiple of the column tile."""
    say(f"head_product K={K} N={N}")
    M = 301
    _, x, w = _operands(M, 16, K, N, K * 1000 + N)
    out = kernels.head_product(x.to(gpu), w.to(gpu))
    torch.cuda.synchronize()
    check(out, ref_head_product(x, w))


@pytest.mark.parametrize("H", [1, 12, 32])
def test_head_counts(gpu, H):
    """The head count only sizes the grid (the reference's presets use 12, 16
    and 32 heads)."""
    say(f"head_product H={H}")
    _, x, w = _operands(257, H, 128, 256, H)
    out = kernels.head_product(x.to(gpu), w.to(gpu))
    torch.cuda.synchronize()
    check(out, ref_head_product(x, w))


def test_strided_output_leaves_gaps_untouched(gpu):
    """y rows wider than H * N: the columns between heads are not written."""
    M, H, K, N = 200, 4, 128, 64
    _, x, w = _operands(M, H, K, N, 5)
    buf = torch.full((M, H, N + 12), 7.0, dtype=torch.bfloat16, device=gpu)
    kernels.head_product(x.to(gpu), w.to(gpu), out=buf[:, :, :N])
    torch.cuda.synchronize()
    check(buf[:, :, :N], ref_head_product(x, w))
    assert bool((buf[:, :, N:] == 7.0).all())


def test_rejects_unbuilt_shapes(gpu):
    x = torch.zeros(4, 2, 96, dtype=torch.bfloat16, device=gpu)
    w = torch.zeros(2, 64, 96, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="K=96"):
        kernels.head_product(x, w)


def test_module_prompt_pass_uses_head_product_and_matches_aten_path(gpu, monkeypatch):
    """A 2 x 300-token bf16 prompt through MLA.forward runs both absorbed
    products on mla_head_product and agrees with the same module on ATen's
    batched products (the path fp32 models take)."""
    from swamla_amd import MLA, MLAConfig

    cfg = MLAConfig(n_embd=1024, max_batch_size=2, max_seq_len=512)
    outs, caches = {}, {}
    for use in (True, False):
        m = MLA(cfg)
        g = torch.Generator().manual_seed(3)
        with torch.no_grad():
            for name, p in m.named_parameters():
                if name.endswith("weight") and not name.startswith("kv_norm"):
                    p.copy_(torch.randn(p.shape, generator=g) * 0.02)
        m.eval().to(torch.bfloat16).to(gpu)
        m.set_inference_mode(True)
        calls = []
        real = kernels.head_product

        def spy(*a, **k):
            calls.append(1)
            return real(*a, **k)

        monkeypatch.setattr(kernels, "head_product", spy)
        monkeypatch.setattr(kernels, "head_product_ok", (lambda K, N: True) if use else (lambda K, N: False))
        gd = torch.Generator(device=gpu).manual_seed(4)
        x = torch.randn(2, 300, 1024, generator=gd, device=gpu).to(torch.bfloat16)
        with torch.no_grad():
            outs[use] = m(x, 0)
        torch.cuda.synchronize()
        assert len(calls) == (2 if use else 0)
        caches[use] = (m.kv_cache[:2, :300].clone(), m.pe_cache[:2, :300].clone())
    assert torch.equal(caches[True][0], caches[False][0]) and torch.equal(caches[True][1], caches[False][1])
    a, b = outs[True].float(), outs[False].float()
    err = (a - b).abs()
    assert not bool((err > 1e-2 + 2e-2 * b.abs()).any()), float(err.max())
