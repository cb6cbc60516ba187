"""mla_decode_attn_noalloc (split partials in the library's fixed per-device
scratch) against mla_decode_attn + mla_merge with caller buffers: the same
kernels, so o_lat and the log-sum-exp must agree bit for bit.  Two calls in
a row on the shared scratch, the second with a smaller input (fewer rows,
shorter rows, fewer splits, and a balanced plan)."""
import pytest
import torch

from swamla_amd import _abi, kernels
from swamla_amd.kernels import LatentCache
from swamla_amd.rope import rope_tables

pytestmark = pytest.mark.gpu

R, P, H = 256, 64, 16
SCALE = 192 ** -0.5


def say(*a):
    print(*a, flush=True)


def _inputs(gpu, fp8, lens, B, S, seed):
    g = torch.Generator().manual_seed(seed)
    rows = len(lens)
    ckv = torch.randn(B, S, R, generator=g).to(torch.bfloat16)
    kpe = torch.randn(B, S, P, generator=g).to(torch.bfloat16)
    if fp8:
        from oracle import latent_ops as lo

        codes, scale = lo.fp8_quantize(ckv.reshape(-1, R))
        cache = LatentCache(codes.view(B, S, R).to(gpu), kpe.to(gpu), scale.view(B, S).to(gpu), R)
    else:
        cache = LatentCache(ckv.to(gpu), kpe.to(gpu), rank=R)
    q_abs = torch.randn(rows, H, R, generator=g).to(torch.bfloat16).to(gpu)
    q_pe = torch.randn(rows, H, P, generator=g).to(torch.bfloat16).to(gpu)
    row_seq = torch.randint(0, B, (rows,), generator=g, dtype=torch.int32).to(gpu)
    kv_len = torch.tensor(lens, dtype=torch.int32).to(gpu)
    rope = torch.randint(0, S, (rows,), generator=g, dtype=torch.int32).to(gpu)
    cos, sin = rope_tables(64, S)
    cos = cos.to(torch.bfloat16)[0, 0, :, :32].contiguous().to(gpu)
    sin = sin.to(torch.bfloat16)[0, 0, :, :32].contiguous().to(gpu)
    return cache, q_abs, q_pe, row_seq, kv_len, rope, cos, sin


def _noalloc(cache, q_abs, q_pe, row_seq, kv_len, rope, cos, sin, n_splits, min_chunk, balance):
    rows = q_abs.shape[0]
    out = torch.full((rows, H, R), float("nan"), dtype=torch.bfloat16, device=q_abs.device)
    lse = torch.full((rows, H), float("nan"), dtype=torch.float32, device=q_abs.device)
    rc = _abi.lib().mla_decode_attn_noalloc(
        q_abs.data_ptr(), q_abs.stride(0), q_abs.stride(1), q_pe.data_ptr(), q_pe.stride(0), q_pe.stride(1),
        cos.data_ptr(), sin.data_ptr(), cos.shape[0], cache.ckv.data_ptr(), cache.kpe.data_ptr(),
        _abi.ptr(cache.scale), cache.ckv.shape[0], cache.ckv.shape[1], row_seq.data_ptr(), kv_len.data_ptr(),
        rope.data_ptr(), None, 1, 0, rows, H, R, P, SCALE, n_splits, min_chunk, balance, out.data_ptr(),
        out.stride(0), out.stride(1), lse.data_ptr(), _abi.DTYPE_BF16, cache.cache_code,
        _abi.stream_handle(q_abs.device))
    _abi.check(rc)
    return out, lse


@pytest.mark.parametrize("fp8", [False, True])
def test_noalloc_decode_equals_workspace_decode(gpu, fp8):
    calls = [
        # rows' lengths, cache (B, S), n_splits, min_chunk, balance_blocks
        ([3000, 17, 1, 2047, 512, 2999, 64, 1500, 777, 2200, 0, 1024], (6, 3008), 8, 64, 0),
        ([900, 5, 333, 64, 700], (4, 1024), 4, 64, 24),
    ]
    for i, (lens, (B, S), ns, mc, bal) in enumerate(calls):
        say(f"noalloc call {i}: fp8={fp8} rows={len(lens)} B={B} S={S} n_splits={ns} min_chunk={mc} balance={bal}")
        args = _inputs(gpu, fp8, lens, B, S, seed=10 + i)
        cache, q_abs, q_pe, row_seq, kv_len, rope, cos, sin = args
        lse_ref = torch.full((len(lens), H), float("nan"), dtype=torch.float32, device=gpu)
        ref = kernels.decode_attention(q_abs, q_pe, cos, sin, cache, SCALE, row_seq=row_seq, kv_len=kv_len,
                                       q_rope_pos=rope, n_splits=ns, min_chunk=mc, balance=bal, lse_out=lse_ref)
        out, lse = _noalloc(*args, ns, mc, bal)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"call {i}: o_lat differs"
        assert torch.equal(lse.view(torch.int32), lse_ref.view(torch.int32)), f"call {i}: lse differs"
        assert bool(torch.isfinite(out.float()).all())


def test_noalloc_rejects_oversize(gpu):
    # 64 rows x 16 splits x 16 heads x 512 channels x 4 B = 32 MiB of partials > 16 MiB
    rows, rank = 64, 512
    q = torch.zeros(rows, H, rank, dtype=torch.bfloat16, device=gpu)
    qp = torch.zeros(rows, H, P, dtype=torch.bfloat16, device=gpu)
    cache = LatentCache.allocate(1, 64, torch.bfloat16, gpu, rank=rank)
    idx = torch.zeros(rows, dtype=torch.int32, device=gpu)
    cos = torch.zeros(64, 32, dtype=torch.bfloat16, device=gpu)
    out = torch.zeros(rows, H, rank, dtype=torch.bfloat16, device=gpu)
    rc = _abi.lib().mla_decode_attn_noalloc(
        q.data_ptr(), q.stride(0), q.stride(1), qp.data_ptr(), qp.stride(0), qp.stride(1), cos.data_ptr(),
        cos.data_ptr(), 64, cache.ckv.data_ptr(), cache.kpe.data_ptr(), None, 1, 64, idx.data_ptr(),
        idx.data_ptr(), idx.data_ptr(), None, 1, 0, rows, H, rank, P, SCALE, 16, 64, 0, out.data_ptr(),
        out.stride(0), out.stride(1), None, _abi.DTYPE_BF16, _abi.DTYPE_BF16, _abi.stream_handle(gpu))
    assert rc == -2
    assert b"scratch" in _abi.lib().mla_last_error()


def test_noalloc_calls_on_two_streams_are_ordered(gpu):
    """The shared scratch on two streams: a call on stream 2, made while the
    device's last call (on stream 1, queued behind a bounded spin) has not
    run, waits for it instead of sharing the area at the same time; both
    results equal the workspace path bit for bit."""
    import time

    lens, (B, S), ns, mc = [1000, 700, 64, 999], (4, 1024), 4, 64
    say(f"noalloc two streams: rows={len(lens)} n_splits={ns}")
    args = _inputs(gpu, False, lens, B, S, seed=77)
    cache, q_abs, q_pe, row_seq, kv_len, rope, cos, sin = args
    lse_ref = torch.full((len(lens), H), float("nan"), dtype=torch.float32, device=gpu)
    ref = kernels.decode_attention(q_abs, q_pe, cos, sin, cache, SCALE, row_seq=row_seq, kv_len=kv_len,
                                   q_rope_pos=rope, n_splits=ns, min_chunk=mc, lse_out=lse_ref)
    s1, s2 = torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)
    torch.cuda.synchronize()
    with torch.cuda.stream(s1):
        torch.cuda._sleep(20_000_000)  # a bounded spin ahead of stream 1's call (milliseconds)
        o1, l1 = _noalloc(*args, ns, mc, 0)
    with torch.cuda.stream(s2):
        o2, l2 = _noalloc(*args, ns, mc, 0)
        done2 = torch.cuda.Event()
        done2.record(s2)
    time.sleep(0.002)  # far longer than the call itself takes
    # stream 2's call is still queued behind stream 1's spin and call
    assert not done2.query()
    torch.cuda.synchronize()
    for o, lse in ((o1, l1), (o2, l2)):
        assert torch.equal(o.view(torch.int16), ref.view(torch.int16))
        assert torch.equal(lse.view(torch.int32), lse_ref.view(torch.int32))
