"""C-ABI and host-side checks that need no GPU: the library loads, exports
every symbol the headers declare, and rejects bad arguments before any HIP
call; the drop-in module mirrors the reference's interface."""
import ctypes
import glob
import os
import re

import pytest
import torch

from swamla_amd import _abi
from swamla_amd.mla import MLA
from oracle.mla_ref import MLAConfig, RefMLA, init_weights

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE = 0x10000  # a 16-byte aligned non-null address; never dereferenced


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[\w]+\s*\*?\s*(mla_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert {"mla_append", "mla_decode_attn", "mla_merge", "mla_abi_version", "mla_last_error"} <= names
    for n in names:
        assert hasattr(lib, n), n
    assert set(_abi.EXPORTED_SYMBOLS) == names


def test_abi_version(lib):
    assert lib.mla_abi_version() == _abi.ABI_VERSION == 6


def _append(lib, **kw):
    args = dict(kv_in=FAKE, in_rs=320, n_tok=4, seq=FAKE, dst=FAKE, rope=FAKE, sp=None, T=1, rope_abs=0,
                w=FAKE, b=FAKE, eps=1e-5, cos=FAKE, sin=FAKE, rope_len=16, ckv=FAKE, kpe=FAKE, scale=None, cb=2,
                cs=16, err=None, in_dt=1, c_dt=1, R=256, P=64, stream=None)
    args.update(kw)
    return lib.mla_append(*args.values())


def _decode(lib, **kw):
    args = dict(qa=FAKE, qa_rs=4096, qa_hs=256, qp=FAKE, qp_rs=3072, qp_hs=192, cos=FAKE, sin=FAKE,
                rope_len=16, ckv=FAKE, kpe=FAKE, scale=None, cb=2, cs=16, row_seq=FAKE, kv_len=FAKE, qrp=FAKE,
                sp=None, T=1, rope_abs=0, n_rows=2, H=16, R=256, P=64, sm=0.07, ns=1, mc=64, bal=0, plan=None,
                o_part=None, lse=None, o=FAKE, o_rs=4096, o_hs=256, lse_out=None, dt=1, c_dt=1, stream=None)
    args.update(kw)
    return lib.mla_decode_attn(*args.values())


@pytest.mark.parametrize(
    "kw,code",
    [
        (dict(R=1025), -2),  # kv_lora_rank 1..1024
        (dict(R=0), -2),
        (dict(P=32), -2),
        (dict(in_dt=0, c_dt=1), -2),
        (dict(in_dt=2, c_dt=2), -2),
        (dict(n_tok=-1), -1),
        (dict(ckv=None), -1),
        (dict(seq=None), -1),
        (dict(c_dt=2), -1),  # fp8 without a scale buffer
        (dict(in_rs=100), -1),
        (dict(R=200, in_rs=300), -1),  # rows hold R_pad = 256 latent channels + 64
        (dict(cs=0), -1),
        (dict(rope_len=0), -1),
        (dict(ckv=FAKE + 8), -3),
        (dict(sp=FAKE), -1),  # both addressing modes
        (dict(seq=None, dst=None, rope=None, sp=FAKE, T=3), -1),  # 4 tokens, 3 per sequence
        (dict(seq=None, dst=None, rope=None, sp=FAKE, T=0), -1),
        (dict(seq=None, dst=None, rope=None, sp=FAKE, T=2, rope_abs=2), -1),
    ],
)
def test_append_rejects(lib, kw, code):
    assert _append(lib, **kw) == code
    assert lib.mla_last_error().decode()


def test_append_zero_tokens_is_a_noop(lib):
    # n_tok = 0 returns before any launch (no GPU needed)
    assert _append(lib, n_tok=0, kv_in=None, seq=None, dst=None, rope=None) == 0
    assert _append(lib, n_tok=0, kv_in=None, seq=None, dst=None, rope=None, sp=FAKE, T=4) == 0


@pytest.mark.parametrize(
    "kw,code",
    [
        (dict(H=8), -2),
        (dict(R=1040), -2),
        (dict(dt=1, c_dt=0), -2),
        (dict(n_rows=70000), -1),
        (dict(ns=0), -1),
        (dict(ns=2000), -1),
        (dict(ns=4), -1),  # no partial buffers
        (dict(mc=0), -1),
        (dict(sm=0.0), -1),
        (dict(sm=float("nan")), -1),
        (dict(o=None), -1),
        (dict(qa_hs=100), -1),
        (dict(R=300, qa_hs=312, o_hs=320), -1),  # head strides cover R_pad = 320
        (dict(c_dt=2), -1),
        (dict(qa=FAKE + 4), -3),
        (dict(o_rs=4100), -3),
        (dict(qp_hs=196), -3),
        (dict(sp=FAKE), -1),
        (dict(row_seq=None, kv_len=None, qrp=None, sp=FAKE, T=3), -1),
        (dict(row_seq=None), -1),
        (dict(bal=-1), -1),
        (dict(bal=70000), -1),
        (dict(bal=1), -1),  # 2 rows need at least 2 workgroups
        (dict(bal=300, n_rows=257), -1),  # a balanced plan covers at most 256 rows
        (dict(bal=256, plan=FAKE + 2), -3),
        (dict(bal=256, cs=(1 << 24) + 1), -2),  # balanced plans cover caches up to 2^24 positions
        (dict(lse_out=FAKE + 2), -3),
    ],
)
def test_decode_rejects(lib, kw, code):
    assert _decode(lib, **kw) == code
    assert lib.mla_last_error().decode()


def _decode_append(lib, **kw):
    args = dict(kv_in=FAKE, in_rs=320, w=FAKE, b=FAKE, eps=1e-5, err=None,
                qa=FAKE, qa_rs=4096, qa_hs=256, qp=FAKE, qp_rs=3072, qp_hs=192, cos=FAKE, sin=FAKE,
                rope_len=16, ckv=FAKE, kpe=FAKE, scale=None, cb=2, cs=16, sp=FAKE, rope_abs=0, n_rows=2,
                H=16, R=256, P=64, sm=0.07, ns=1, mc=64, bal=0, plan=None, o_part=None, lse=None, o=FAKE,
                o_rs=4096, o_hs=256, lse_out=None, dt=1, c_dt=1, stream=None)
    args.update(kw)
    return lib.mla_decode_attn_append(*args.values())


@pytest.mark.parametrize(
    "kw,code",
    [
        (dict(dt=0, c_dt=0), -2),  # fp32 models keep the separate append
        (dict(c_dt=0), -2),
        (dict(H=8), -2),
        (dict(sp=None), -1),  # dense addressing only
        (dict(kv_in=None), -1),
        (dict(w=None), -1),
        (dict(in_rs=300), -1),
        (dict(kv_in=FAKE + 4), -3),
        (dict(in_rs=322), -3),
        (dict(w=FAKE + 2), -3),
        (dict(R=512, in_rs=576, qa_hs=512, o_hs=512, kv_in=FAKE + 8), -3),  # 8 channels a lane: 16-byte loads
        (dict(R=512, in_rs=580, qa_hs=512, o_hs=512), -3),
        (dict(c_dt=2), -1),  # fp8 without a scale buffer
        (dict(ns=4), -1),
        (dict(o=None), -1),
        (dict(rope_abs=3), -1),
        (dict(qa=FAKE + 4), -3),
        (dict(bal=1), -1),
        (dict(bal=256, plan=FAKE + 1), -3),
    ],
)
def test_decode_append_rejects(lib, kw, code):
    assert _decode_append(lib, **kw) == code
    assert "mla_decode_attn_append" in lib.mla_last_error().decode() or code == -2


def _prefill(lib, **kw):
    args = dict(qa=FAKE, qa_rs=4096, qa_hs=256, qp=FAKE, qp_rs=3072, qp_hs=192, cos=FAKE, sin=FAKE,
                rope_len=16, ckv=FAKE, kpe=FAKE, scale=None, cb=2, cs=16, sp=FAKE, T=4, rope_abs=0, n_rows=8,
                H=16, R=256, P=64, sm=0.07, o=FAKE, o_rs=4096, o_hs=256, dt=1, c_dt=1, stream=None)
    args.update(kw)
    return lib.mla_prefill_attn(*args.values())


@pytest.mark.parametrize(
    "kw,code",
    [
        (dict(dt=0, c_dt=0), -2),  # fp32 models use the per-row path
        (dict(H=8), -2),
        (dict(sp=None), -1),  # dense addressing only
        (dict(T=3), -1),  # 8 rows are not a multiple of 3
        (dict(T=0), -1),
        (dict(n_rows=70000 * 4, T=4), -1),  # more than 65535 sequences
        (dict(c_dt=2), -1),
        (dict(o=None), -1),
        (dict(qa=FAKE + 4), -3),
        (dict(cos=FAKE + 4), -3),
    ],
)
def test_prefill_rejects(lib, kw, code):
    assert _prefill(lib, **kw) == code
    assert lib.mla_last_error().decode()


def test_prefill_zero_rows_is_a_noop(lib):
    assert _prefill(lib, n_rows=0, qa=None, qp=None) == 0


def test_decode_append_zero_rows_is_a_noop(lib):
    assert _decode_append(lib, n_rows=0, kv_in=None, qa=None, qp=None) == 0


def _merge(lib, **kw):
    args = dict(o_part=FAKE, lse=FAKE, row_seq=FAKE, kv_len=FAKE, sp=None, T=1, cb=2, cs=64, n_rows=2, H=16,
                R=256, ns=4, mc=64, plan=None, o=FAKE, o_rs=4096, o_hs=256, lse_out=None, dt=1, stream=None)
    args.update(kw)
    return lib.mla_merge(*args.values())


def test_merge_rejects_and_noop(lib):
    assert _merge(lib, ns=1) == 0
    assert _merge(lib, R=1025) == -2
    assert _merge(lib, o_part=None) == -1
    assert _merge(lib, dt=2) == -2
    assert _merge(lib, o_part=FAKE + 4) == -3
    assert _merge(lib, kv_len=None) == -1
    assert _merge(lib, row_seq=None) == -1  # the decode call's cache rows
    assert _merge(lib, sp=FAKE) == -1
    assert _merge(lib, cs=0) == -1
    assert _merge(lib, plan=FAKE + 2) == -3


def _linear(lib, **kw):
    args = dict(x=FAKE, x_rs=1024, x_bs=0, w=FAKE, w_rs=1024, w_bs=0, bias=None, bias_bs=0, y=FAKE,
                y_rs=64, y_bs=0, M=32, N=64, K=1024, batch=1, dt=1, stream=None)
    args.update(kw)
    return lib.mla_linear(*args.values())


@pytest.mark.parametrize(
    "kw,code",
    [
        (dict(dt=0), -2),
        (dict(M=129), -2),
        (dict(N=40), -2),
        (dict(K=100), -2),
        (dict(K=0), -2),
        (dict(batch=-1), -1),
        (dict(x=None), -1),
        (dict(x_rs=512), -1),
        (dict(y_rs=32), -1),
        (dict(x=FAKE + 8), -3),
        (dict(w_rs=1028), -3),
        (dict(x_bs=4), -3),
    ],
)
def test_linear_rejects(lib, kw, code):
    assert _linear(lib, **kw) == code
    assert lib.mla_last_error().decode()


def test_pack_weight_and_packed_linear_reject(lib):
    assert lib.mla_pack_weight(FAKE, 1024, 48, 1024, FAKE, 0, None) == -2  # fp32
    assert lib.mla_pack_weight(FAKE, 1024, 44, 1024, FAKE, 1, None) == -2  # N % 8
    assert lib.mla_pack_weight(FAKE, 1024, 48, 1000, FAKE, 1, None) == -2  # K % 64
    assert lib.mla_pack_weight(FAKE, 512, 48, 1024, FAKE, 1, None) == -1  # row stride < K
    assert lib.mla_pack_weight(None, 1024, 48, 1024, FAKE, 1, None) == -1
    assert lib.mla_pack_weight(FAKE + 8, 1024, 48, 1024, FAKE, 1, None) == -3
    assert lib.mla_pack_weight(FAKE, 1028, 48, 1024, FAKE, 1, None) == -3
    assert lib.mla_pack_weight(FAKE, 1024, 0, 1024, None, 1, None) == 0  # empty
    args = dict(x=FAKE, x_rs=1024, wp=FAKE, bias=None, y=FAKE, y_rs=64, M=32, N=64, K=1024, adv=None, n_adv=0, dt=1,
                stream=None)

    def lp(**kw):
        a = dict(args)
        a.update(kw)
        return lib.mla_linear_packed(*a.values())

    assert lp(dt=0) == -2
    assert lp(M=129) == -2
    assert lp(N=60) == -2
    assert lp(K=768) == -2
    assert lp(K=4096) == -2
    assert lp(x=None) == -1
    assert lp(x_rs=512) == -1
    assert lp(y_rs=32) == -1
    assert lp(x=FAKE + 8) == -3
    assert lp(x_rs=1028) == -3
    assert lp(bias=FAKE + 1) == -3
    assert lp(M=0, x=None, wp=None, y=None) == 0
    # the position advance: 1 to 512 entries, 4-byte aligned, a non-empty product
    assert lp(adv=FAKE, n_adv=0) == -1
    assert lp(adv=FAKE, n_adv=513) == -1
    assert lp(adv=FAKE, n_adv=4, M=0, x=None, wp=None, y=None) == -1
    assert "advance" in lib.mla_last_error().decode()
    assert lp(adv=FAKE + 2, n_adv=4) == -3
    assert "mla_linear_packed" in lib.mla_last_error().decode() or lp(M=129) == -2


def test_linear_empty_is_a_noop(lib):
    assert _linear(lib, M=0, x=None, w=None, y=None) == 0
    assert _linear(lib, batch=0, x=None, w=None, y=None) == 0


def _merge_project(lib, **kw):
    args = dict(o_part=FAKE, lse=FAKE, o_lat=FAKE, o_rs=4096, o_hs=256, kv_len=FAKE, row_seq=FAKE, sp=None, T=1,
                cb=4, cs=64, n_rows=8, H=16, R=256, ns=4, mc=64, plan=None, w=FAKE, w_rs=256, w_hs=65536, Dv=128,
                y=FAKE, y_rs=2048, y_hs=128, dt=1, stream=None)
    args.update(kw)
    return lib.mla_merge_project(*args.values())


@pytest.mark.parametrize(
    "kw,code",
    [
        (dict(dt=0), -2),
        (dict(Dv=64), -2),
        (dict(R=600), -2),
        (dict(ns=0), -1),
        (dict(o_part=None), -1),
        (dict(row_seq=None), -1),
        (dict(w=None), -1),
        (dict(cs=0), -1),
        (dict(o_hs=128), -1),
        (dict(o_lat=FAKE + 8), -3),
        (dict(w_rs=260), -3),
        (dict(sp=FAKE), -1),
        (dict(plan=FAKE + 2), -3),
    ],
)
def test_merge_project_rejects(lib, kw, code):
    assert _merge_project(lib, **kw) == code
    assert lib.mla_last_error().decode()


def test_merge_project_single_split_needs_no_partials(lib):
    # validation passes without partial buffers when n_splits == 1 (n_rows = 0: no launch)
    assert _merge_project(lib, ns=1, o_part=None, lse=None, n_rows=0) == 0


def test_python_check_raises_with_message(lib):
    rc = _append(lib, R=1088)
    with pytest.raises(_abi.SwamlaError, match="UNSUPPORTED.*R=1088"):
        _abi.check(rc)
    with pytest.raises(RuntimeError):
        _abi.check(rc)


# ---------------------------------------------------------------- module
def small_cfg(**kw):
    d = dict(n_embd=128, max_batch_size=2, max_seq_len=32)
    d.update(kw)
    return MLAConfig(**d)


def test_state_dict_interchanges_with_reference():
    ref = RefMLA(small_cfg())
    init_weights(ref, 0, ln_random=True)
    ours = MLA(small_cfg())
    ours.load_state_dict(ref.state_dict())
    assert list(ours.state_dict().keys()) == list(ref.state_dict().keys())
    for k, v in ref.state_dict().items():
        assert torch.equal(ours.state_dict()[k], v)
    assert ours.softmax_scale == ref.softmax_scale == 192 ** -0.5


def test_rope_table_bitwise_equal_to_reference():
    ref = RefMLA(small_cfg(max_seq_len=300)).to(torch.bfloat16)
    ours = MLA(small_cfg(max_seq_len=300)).to(torch.bfloat16)
    assert torch.equal(ours.rope.cos_cached, ref.rope.cos_cached)
    assert torch.equal(ours.rope.sin_cached, ref.rope.sin_cached)
    cos, sin = ours.rope.half_tables()
    assert cos.shape == (300, 32) and torch.equal(cos, ref.rope.cos_cached[0, 0, :, :32])


def test_rope_extend_matches_reference_growth():
    """MLA.rope.extend grows the table like positional_encoding.py:64-86: the
    same fp32 table as the restatement's growth, bit for bit, in fp32 even in a
    bf16 module, with max_seq_len moved to the new length."""
    ref = RefMLA(small_cfg(max_seq_len=16)).to(torch.bfloat16)
    ours = MLA(small_cfg(max_seq_len=16)).to(torch.bfloat16)
    ours.rope.half_tables()
    ref.rope(torch.zeros(1, 1, 50, 64, dtype=torch.bfloat16))
    ours.rope.extend(50)
    assert ours.rope.max_seq_len == ref.rope.max_seq_len == 50
    assert ours.rope.cos_cached.dtype == torch.float32
    assert torch.equal(ours.rope.cos_cached, ref.rope.cos_cached)
    assert torch.equal(ours.rope.sin_cached, ref.rope.sin_cached)
    cos, _ = ours.rope.half_tables()
    assert cos.shape == (50, 32) and cos.dtype == torch.float32
    assert len(ours.rope._retired) == 1  # the old half tables stay alive
    ours.rope.extend(20)  # never shrinks
    assert ours.rope.max_seq_len == 50


def test_inference_mode_allocation_and_clear():
    m = MLA(small_cfg()).to(torch.bfloat16)
    m.set_inference_mode(True)  # works directly (the reference's raises KeyError)
    assert m.kv_cache.shape == (2, 32, 256) and m.kv_cache.dtype == torch.bfloat16
    assert m.pe_cache.shape == (2, 32, 64) and m.pe_cache.dtype == torch.bfloat16
    assert "kv_cache" not in m.state_dict()  # persistent=False as in mla.py:207-215
    m.set_inference_mode(False)
    assert not hasattr(m, "kv_cache")
    m.set_inference_mode(True)
    m.clear_cache()
    assert m.kv_cache is None and m.inference_mode is False
    m.set_inference_mode(True)
    assert m.kv_cache is not None


def test_fp8_cache_scale_stays_fp32():
    m = MLA(small_cfg(), cache_dtype="fp8_e4m3")
    m.set_inference_mode(True)
    assert m.kv_cache.dtype == torch.uint8 and m.kv_scale.dtype == torch.float32
    m.to(torch.bfloat16)
    assert m.kv_cache.dtype == torch.uint8 and m.kv_scale.dtype == torch.float32
    assert m.pe_cache.dtype == torch.bfloat16


def test_no_cpu_fallback():
    m = MLA(small_cfg()).eval()
    m.set_inference_mode(True)
    with torch.no_grad(), pytest.raises(RuntimeError, match="GPU only"):
        m(torch.randn(1, 1, 128), 0)


def test_unsupported_paths_raise():
    m = MLA(small_cfg()).eval()
    x = torch.randn(1, 2, 128)
    with pytest.raises(NotImplementedError):
        m(x, 0, mask=torch.zeros(2, 2))
    with pytest.raises(NotImplementedError):
        m(x, 0, position_ids=torch.zeros(1, 2, dtype=torch.long))
    with pytest.raises(NotImplementedError):
        m(x.requires_grad_(), 0)


def _brute_balanced_chunk(lens, n_splits, min_chunk, target):
    """The definition, searched directly: the smallest multiple of 64 tokens
    >= min_chunk with every row in at most n_splits pieces and at most
    target workgroups in all (an empty row takes one)."""
    c = 64 * max(1, -(-min_chunk // 64))
    while True:
        pieces = [(-(-L // c) if L > 0 else 1) for L in lens]
        if max([p for p, L in zip(pieces, lens) if L > 0] or [0]) <= n_splits and sum(pieces) <= target:
            return c
        c += 64


@pytest.mark.parametrize("seed", range(6))
def test_balanced_chunk_matches_its_definition(seed):
    import random

    from swamla_amd import kernels

    rng = random.Random(seed)
    for _ in range(40):
        n = rng.randint(1, 64)
        hi = rng.choice([70, 700, 17000, 140000])
        lens = [rng.choice([0, rng.randint(1, hi), rng.randint(1, 64)]) for _ in range(n)]
        target = rng.choice([n, n + 1, 64, 256, 1000]) if n <= 64 else 256
        target = max(target, n)
        n_splits = rng.choice([1, 4, 16, 129, 1024])
        min_chunk = rng.choice([1, 64, 100, 256, 4096])
        want = _brute_balanced_chunk(lens, n_splits, min_chunk, target)
        assert kernels.balanced_chunk(lens, n_splits, min_chunk, target) == want, (lens, n_splits, min_chunk, target)


def test_decode_blocks_per_cu_rejects(lib):
    """Argument checks come before any HIP call."""
    bf, f32, fp8 = _abi.DTYPE_BF16, _abi.DTYPE_F32, _abi.DTYPE_FP8
    assert lib.mla_decode_blocks_per_cu(bf, bf, 0, 0) == -2
    assert lib.mla_decode_blocks_per_cu(bf, bf, 1025, 0) == -2
    assert lib.mla_decode_blocks_per_cu(f32, fp8, 256, 0) == -2
    assert lib.mla_decode_blocks_per_cu(fp8, fp8, 256, 0) == -2
    assert lib.mla_decode_blocks_per_cu(bf, bf, 256, 2) == -1
    assert "fused" in lib.mla_last_error().decode()


def test_balanced_chunk_examples_and_rejects(lib):
    from swamla_amd import kernels

    # uniform rows: the static plan's tile count per workgroup
    assert kernels.balanced_chunk([4224] * 32, 16, 256, 256) == 9 * 64
    # one long row among short ones takes many workgroups
    c = kernels.balanced_chunk([16000] + [100] * 15, 256, 64, 256)
    assert -(-16000 // c) + 15 <= 256 and c <= 128
    arr = (ctypes.c_int32 * 4)(1, 2, 3, 4)
    assert lib.mla_balanced_chunk(arr, 4, 8, 64, 3) == -1  # fewer workgroups than rows
    assert lib.mla_balanced_chunk(arr, 4, 0, 64, 8) == -1
    assert lib.mla_balanced_chunk(None, 4, 8, 64, 8) == -1
    assert lib.mla_balanced_chunk(arr, 0, 8, 64, 8) == 64
    big = (ctypes.c_int32 * 2)(1 << 24, (1 << 24) + 1)
    assert lib.mla_balanced_chunk(big, 1, 8, 64, 8) > 0
    assert lib.mla_balanced_chunk(big, 2, 8, 64, 8) == -1


def test_probes_reject(lib):
    """The measurement kernels behind bench.py's ceiling legs validate like
    the product entry points (no HIP call on a bad argument)."""
    E_ARG, E_UNS, E_MIS = -1, -2, -3  # SWAMLA_ERR_INVALID_ARG / _UNSUPPORTED / _MISALIGNED
    assert lib.mla_probe_read(None, 1024, FAKE, 8, None) == E_ARG
    assert lib.mla_probe_read(FAKE, 1000, FAKE, 8, None) == E_ARG  # not a multiple of 16
    assert lib.mla_probe_read(FAKE, 1024, FAKE, 0, None) == E_ARG
    assert lib.mla_probe_read(FAKE + 8, 1024, FAKE, 8, None) == E_MIS

    def stream(**kw):
        a = dict(ckv=FAKE, kpe=FAKE, scale=None, cb=2, cs=64, sp=FAKE, n_rows=2, R=256, ns=4, mc=16, c_dt=1,
                 sink=FAKE, stream=None)
        a.update(kw)
        return lib.mla_probe_cache_stream(*a.values())

    assert stream(R=600) == E_UNS
    assert stream(c_dt=0) == E_UNS
    assert stream(c_dt=2) == E_ARG  # fp8 without scales
    assert stream(sp=None) == E_ARG
    assert stream(ns=0) == E_ARG
    assert stream(ckv=FAKE + 8) == E_MIS


def test_32_heads_only_where_built(lib):
    """32 heads in one launch: bf16 model (bf16 or e4m3 cache) with R_pad <=
    256; any other combination, and other head counts, are rejected before
    any HIP call."""
    E_UNS = -2
    assert _decode(lib, H=32, dt=0, c_dt=0) == E_UNS              # fp32 model
    assert _decode(lib, H=32, R=300, qa_rs=32 * 320, qa_hs=320, o_rs=32 * 320, o_hs=320) == E_UNS
    assert _decode(lib, H=48) == E_UNS and _decode(lib, H=8) == E_UNS
    assert "32" in lib.mla_last_error().decode()
