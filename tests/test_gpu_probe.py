"""GPU checks of the measurement kernels behind bench.py's roofline ceiling
(mla_probe_read, mla_probe_cache_stream): they read what they claim to.

The read probe's checksum is exact: thread t folds (XOR) every 16-byte word
i = t, t + nt, ... of the buffer.  The stream probe folds, per wave, the first
16 bytes its lane receives of every sub-tile; its checksum must be
reproducible and must change when a cache row inside a streamed split
changes, and not when a row beyond every row's length does."""
import numpy as np
import pytest
import torch

from swamla_amd import _abi, kernels
from swamla_amd.kernels import LatentCache

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def test_read_probe_checksum_exact(gpu):
    say("probe: read checksum")
    lib = _abi.lib()
    nbytes, grid = (1 << 20) + 16 * 77, 8
    g = torch.Generator(device=gpu).manual_seed(1)
    buf = torch.randint(-(1 << 31), (1 << 31) - 1, (nbytes // 4,), generator=g, device=gpu, dtype=torch.int64)
    buf = buf.to(torch.int32)
    sink = torch.zeros(grid * 256, dtype=torch.int32, device=gpu)
    _abi.check(lib.mla_probe_read(buf.data_ptr(), nbytes, sink.data_ptr(), grid,
                                  torch.cuda.current_stream(gpu).cuda_stream))
    torch.cuda.synchronize()
    words = buf.cpu().numpy().view(np.uint32).reshape(-1, 4)
    per16 = words[:, 0] ^ words[:, 1] ^ words[:, 2] ^ words[:, 3]
    nt = grid * 256
    want = np.zeros(nt, np.uint32)
    for t in range(nt):
        want[t] = np.bitwise_xor.reduce(per16[t::nt]) if t < per16.size else 0
    assert np.array_equal(sink.cpu().numpy().view(np.uint32), want)


def test_stream_probe_reads_the_attended_rows(gpu):
    say("probe: cache stream")
    lib = _abi.lib()
    B, S, R, P = 4, 2048, 256, 64
    g = torch.Generator(device=gpu).manual_seed(2)
    cache = LatentCache(torch.randn(B, S, R, generator=g, device=gpu).to(torch.bfloat16),
                        torch.randn(B, S, P, generator=g, device=gpu).to(torch.bfloat16))
    sp = torch.tensor([1999, 700, 15, 1024], dtype=torch.int32, device=gpu)  # rows attend [0, sp + 1)
    n_splits, min_chunk = 4, 64
    hc = torch.cuda.current_stream(gpu).cuda_stream

    def run():
        sink = torch.zeros(n_splits * B * 256, dtype=torch.int32, device=gpu)
        _abi.check(lib.mla_probe_cache_stream(cache.ckv.data_ptr(), cache.kpe.data_ptr(), None, B, S,
                                              sp.data_ptr(), B, R, n_splits, min_chunk, _abi.DTYPE_BF16,
                                              sink.data_ptr(), hc))
        torch.cuda.synchronize()
        return sink.cpu()

    base = run()
    assert torch.equal(base, run())
    assert int((base != 0).sum()) > 0
    # the first row of every sub-tile feeds the checksum: changing row 0's
    # first latent chunk of sequence 0 changes it; a row past every length
    # (position 2040 of sequence 1, which attends 701 tokens) does not
    saved = cache.ckv[0, 0].clone()
    cache.ckv[0, 0, :8] += 1.0
    assert not torch.equal(base, run())
    cache.ckv[0, 0] = saved
    assert torch.equal(base, run())
    cache.ckv[1, 2040] += 1.0
    assert torch.equal(base, run())
