"""Tensor-level wrappers of the three C-ABI kernels.

Each wrapper checks shapes, dtypes and devices of torch tensors, then passes
raw pointers, strides and torch's current HIP stream to the library.  They
allocate only the outputs they return (callers that cannot allocate pass
``out=`` / workspace tensors).  There is no CPU or eager fallback: a tensor
that is not on a ROCm device is an error.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _abi

R, P, H = 256, 64, 16  # R: the default kv_lora_rank (any 1..MAX_RANK is built)
# Heads one decode launch takes: 16, or 32 for a bf16 model with R_pad <= 256
# (each wave serves two head groups from one stream of the cache).
DECODE_HEADS = (16, 32)
MAX_RANK = 1024  # the append, the merge and decode attention (the VALU kernel above MFMA_MAX_RANK)
MFMA_MAX_RANK = 512  # the MFMA decode kernel, the fused decode step, merge_project and the stream probe


def padded_rank(rank: int) -> int:
    """Latent channels stored per token for kv_lora_rank ``rank``: R_pad =
    64 * ceil(rank / 64) (the kernels' row layout; channels >= rank are 0)."""
    return 64 * -(-int(rank) // 64)


def _need_gpu(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"swamla_amd kernels run on the GPU only; got a tensor on {t.device}"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    assert dev is not None
    return dev


def _i32(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.int32 or not t.is_contiguous() or t.dim() != 1:
        raise TypeError(f"{name} must be a contiguous 1-D int32 tensor")
    return t


@dataclass
class LatentCache:
    """Latent KV cache of one MLA layer.

    ckv   [B, S, R_pad]  model dtype (bf16 / fp32) or uint8 e4m3fn codes;
                         channels rank .. R_pad-1 hold zeros
    kpe   [B, S, P]      model dtype
    scale [B, S]         fp32 per-token scale (e4m3 caches only)
    rank                 kv_lora_rank R (R_pad = padded_rank(R))
    """

    ckv: torch.Tensor
    kpe: torch.Tensor
    scale: Optional[torch.Tensor] = None
    rank: int = R

    @property
    def rank_pad(self) -> int:
        return padded_rank(self.rank)

    @property
    def is_fp8(self) -> bool:
        return self.ckv.dtype == torch.uint8

    @property
    def model_dtype(self) -> torch.dtype:
        return self.kpe.dtype

    @property
    def cache_code(self) -> int:
        return _abi.DTYPE_FP8 if self.is_fp8 else _abi.dtype_code(self.ckv.dtype)

    def validate(self) -> None:
        c, p = self.ckv, self.kpe
        if c.dim() != 3 or p.dim() != 3 or c.shape[:2] != p.shape[:2]:
            raise ValueError(f"cache shapes {tuple(c.shape)} / {tuple(p.shape)} disagree")
        if not 1 <= self.rank <= MAX_RANK:
            raise ValueError(f"kv_lora_rank {self.rank} outside 1..{MAX_RANK}")
        if c.shape[2] != self.rank_pad or p.shape[2] != P:
            raise ValueError(f"cache last dims must be R_pad={self.rank_pad} (rank {self.rank}), P={P}")
        if not (c.is_contiguous() and p.is_contiguous()):
            raise ValueError("cache buffers must be contiguous")
        if self.is_fp8:
            s = self.scale
            if s is None or s.dtype != torch.float32 or tuple(s.shape) != tuple(c.shape[:2]):
                raise ValueError("e4m3 cache needs a float32 scale of shape [B, S]")
            if not s.is_contiguous():
                raise ValueError("scale must be contiguous")
        elif c.dtype != p.dtype:
            raise ValueError(f"latent cache dtype {c.dtype} != k_pe dtype {p.dtype}")

    @staticmethod
    def allocate(batch: int, seq: int, dtype: torch.dtype, device, fp8: bool = False, rank: int = R) -> "LatentCache":
        rp = padded_rank(rank)
        if fp8:
            return LatentCache(
                torch.zeros(batch, seq, rp, dtype=torch.uint8, device=device),
                torch.zeros(batch, seq, P, dtype=dtype, device=device),
                torch.zeros(batch, seq, dtype=torch.float32, device=device),
                rank,
            )
        return LatentCache(
            torch.zeros(batch, seq, rp, dtype=dtype, device=device),
            torch.zeros(batch, seq, P, dtype=dtype, device=device),
            rank=rank,
        )


def pad_rank(t: torch.Tensor, rank: int, dim: int = -1) -> torch.Tensor:
    """``t`` with dimension ``dim`` (of size rank) zero-padded to
    padded_rank(rank); ``t`` itself when no padding is needed."""
    rp = padded_rank(rank)
    if t.shape[dim] == rp:
        return t
    if t.shape[dim] != rank:
        raise ValueError(f"dimension {dim} has {t.shape[dim]} entries, expected {rank} or {rp}")
    shape = list(t.shape)
    shape[dim] = rp
    out = torch.zeros(shape, dtype=t.dtype, device=t.device)
    out.narrow(dim, 0, rank).copy_(t)
    return out


def _addressing(n, arrays, start_pos, per_seq, names):
    """Validate one of the two addressing modes; returns the ctypes pointers."""
    if start_pos is not None:
        if any(a is not None for a in arrays):
            raise ValueError("pass either start_pos or the per-entry index arrays, not both")
        _i32(start_pos, "start_pos")
        if per_seq < 1 or n % per_seq != 0 or start_pos.numel() != n // per_seq:
            raise ValueError(f"start_pos has {start_pos.numel()} entries for {n} entries of {per_seq} per sequence")
        return [None] * len(arrays), start_pos.data_ptr()
    out = []
    for name, t in zip(names, arrays):
        if t is None:
            out.append(None)
            continue
        _i32(t, name)
        if t.numel() != n:
            raise ValueError(f"{name} has {t.numel()} entries, expected {n}")
        out.append(t.data_ptr())
    return out, None


def append(
    kv: torch.Tensor,
    cache: LatentCache,
    ln_w: torch.Tensor,
    ln_b: torch.Tensor,
    eps: float,
    cos_tab: torch.Tensor,
    sin_tab: torch.Tensor,
    *,
    seq_idx: Optional[torch.Tensor] = None,
    dst_pos: Optional[torch.Tensor] = None,
    rope_pos: Optional[torch.Tensor] = None,
    start_pos: Optional[torch.Tensor] = None,
    tokens_per_seq: int = 1,
    rope_abs: bool = False,
    err_flag: Optional[torch.Tensor] = None,
) -> None:
    """Fused kv_norm + RoPE(k_pe) + (e4m3) + scatter of ``kv`` rows.

    kv: [N, >=R_pad+P] with unit stride in the last dim: the latent part in
    channels [0, R) (R .. R_pad-1 ignored) and k_pe at [R_pad, R_pad+P) (the
    wkv_a output for R = R_pad; the module's padded product otherwise).
    ln_w / ln_b: [R] or [R_pad] (an [R] pair is padded here, one copy).
    Addressing: explicit (seq_idx, dst_pos, rope_pos) or dense (start_pos
    [N / tokens_per_seq]).  Reference: models/mla.py:307-323, :409-414.
    """
    cache.validate()
    dev = _need_gpu(kv, ln_w, ln_b, cos_tab, sin_tab, cache.ckv, seq_idx, dst_pos, rope_pos, start_pos)
    rk, rp = cache.rank, cache.rank_pad
    if kv.dim() != 2 or kv.stride(1) != 1 or kv.shape[1] < rp + P:
        raise ValueError(f"kv must be [N, R_pad+P = {rp + P}] with unit last-dim stride")
    dt = cache.model_dtype
    if kv.dtype != dt or ln_w.dtype != dt or ln_b.dtype != dt or cos_tab.dtype != dt or sin_tab.dtype != dt:
        raise TypeError(f"kv / LayerNorm / RoPE tensors must all be {dt}")
    n = kv.shape[0]
    (p_seq, p_dst, p_rope), p_sp = _addressing(
        n, (seq_idx, dst_pos, rope_pos), start_pos, tokens_per_seq, ("seq_idx", "dst_pos", "rope_pos"))
    if not (ln_w.is_contiguous() and ln_b.is_contiguous() and ln_w.numel() in (rk, rp) and ln_b.numel() in (rk, rp)):
        raise ValueError("LayerNorm weight / bias must be contiguous [R] or [R_pad]")
    ln_w, ln_b = pad_rank(ln_w.reshape(-1), rk), pad_rank(ln_b.reshape(-1), rk)
    if cos_tab.dim() != 2 or cos_tab.shape[1] != P // 2 or cos_tab.shape != sin_tab.shape:
        raise ValueError("RoPE tables must be [S, P/2]")
    if not (cos_tab.is_contiguous() and sin_tab.is_contiguous()):
        raise ValueError("RoPE tables must be contiguous")
    lib = _abi.lib()
    _abi.check(
        lib.mla_append(
            kv.data_ptr(), kv.stride(0), n, p_seq, p_dst, p_rope, p_sp, int(tokens_per_seq), int(bool(rope_abs)),
            ln_w.data_ptr(), ln_b.data_ptr(), float(eps), cos_tab.data_ptr(), sin_tab.data_ptr(),
            cos_tab.shape[0], cache.ckv.data_ptr(), cache.kpe.data_ptr(), _abi.ptr(cache.scale),
            cache.ckv.shape[0], cache.ckv.shape[1], _abi.ptr(err_flag),
            _abi.dtype_code(dt), cache.cache_code, rk, P, _abi.stream_handle(dev),
        )
    )


def plan_splits(n_rows: int, max_len: int, num_cus: int = 256, blocks_per_cu: int = 1,
                min_chunk: int = 256) -> tuple[int, int]:
    """Host heuristic for the split-KV plan: about ``blocks_per_cu`` blocks
    per CU (fewer, longer blocks amortise each block's fixed cost).

    Returns (n_splits, min_chunk).  The kernels derive each row's own split
    count from its length on the device, so ``max_len`` may be an upper bound.
    """
    if n_rows <= 0:
        return 1, min_chunk
    target = max(1, (num_cus * blocks_per_cu + n_rows - 1) // n_rows)
    by_len = max(1, (max_len + min_chunk - 1) // min_chunk)
    return int(max(1, min(target, by_len, 1024))), int(min_chunk)


_BLOCKS_PER_CU: dict = {}


def decode_blocks_per_cu(model_dtype: torch.dtype, fp8_cache: bool, rank: int, fused: bool,
                         device: torch.device) -> int:
    """Decode workgroups one CU holds at once for this kernel instance
    (mla_decode_blocks_per_cu; cached per device): 1 for a bf16 cache, 3 for
    an e4m3 cache at ranks up to 256.  Split plans target CUs x this."""
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    cache = _abi.DTYPE_FP8 if fp8_cache else _abi.dtype_code(model_dtype)
    key = (idx, _abi.dtype_code(model_dtype), cache, int(rank), bool(fused))
    n = _BLOCKS_PER_CU.get(key)
    if n is None:
        with torch.cuda.device(idx):
            n = _abi.lib().mla_decode_blocks_per_cu(key[1], cache, int(rank), int(bool(fused)))
        if n < 1:
            _abi.check(n)
        _BLOCKS_PER_CU[key] = n
    return n


BALANCE_MAX_ROWS = 256  # rows a balanced plan covers (mla_decode_attn)


def balanced_splits(n_rows: int, num_cus: int = 256, blocks_per_cu: int = 1) -> tuple[int, int]:
    """Host side of a length-balanced plan (ragged batches): returns
    (balance_blocks, n_splits) for decode_attention's ``balance`` and
    ``n_splits``: one workgroup per slot (num_cus x blocks_per_cu slots), and
    a per-row split cap of 4 * ceil(slots / n_rows), so one row may take
    several times its share while the partial buffers stay near 4 * slots
    splits.  (0, 0) when the batch has more rows than a balanced plan
    covers."""
    slots = num_cus * max(1, blocks_per_cu)
    if n_rows <= 0 or n_rows > min(slots, BALANCE_MAX_ROWS):
        return 0, 0
    return int(slots), int(min(1024, 4 * -(-slots // n_rows)))


def balanced_chunk(lens, n_splits: int, min_chunk: int, balance_blocks: int) -> int:
    """The chunk (tokens) a balanced decode launch chooses for these row
    lengths (host integers, clamped to the cache); mla_balanced_chunk."""
    arr = (ctypes.c_int32 * max(len(lens), 1))(*[int(v) for v in lens])
    c = int(_abi.lib().mla_balanced_chunk(arr, len(lens), int(n_splits), int(min_chunk), int(balance_blocks)))
    if c < 0:
        raise _abi.SwamlaError(c, _abi.lib().mla_last_error().decode())
    return c


@dataclass
class DecodeWorkspace:
    """Split-KV partial buffers: o_part [rows, splits, H, R_pad], lse [rows,
    splits, H], and ``plan`` (int32 [1]): the chunk a balanced decode launch
    chose, read by the merge that follows it."""

    o_part: torch.Tensor
    lse_part: torch.Tensor
    plan: torch.Tensor

    @staticmethod
    def allocate(n_rows: int, n_splits: int, device, rank: int = R, heads: int = H) -> "DecodeWorkspace":
        rows = max(n_rows, 1)
        return DecodeWorkspace(
            torch.empty(rows, n_splits, heads, padded_rank(rank), dtype=torch.float32, device=device),
            torch.empty(rows, n_splits, heads, dtype=torch.float32, device=device),
            torch.zeros(1, dtype=torch.int32, device=device),
        )

    def fits(self, n_rows: int, n_splits: int, rank: int = R, heads: int = H) -> bool:
        return (self.o_part.shape[0] >= n_rows and self.o_part.shape[1] == n_splits
                and self.o_part.shape[2] == heads and self.o_part.shape[3] == padded_rank(rank))


@dataclass
class FusedAppend:
    """The append that decode_attention folds into its launch for a one-token
    step: row r's new token ``kv[r]`` ([rows, >=R_pad+P] bf16, unit last
    stride, laid out as for append()) goes through kv_norm (``ln_w``,
    ``ln_b``: [R] or [R_pad]) and RoPE and is written at ``start_pos[r]``
    before row r attends."""

    kv: torch.Tensor
    ln_w: torch.Tensor
    ln_b: torch.Tensor
    eps: float
    err_flag: Optional[torch.Tensor] = None


def decode_attention(
    q_abs: torch.Tensor,
    q_pe: torch.Tensor,
    cos_tab: torch.Tensor,
    sin_tab: torch.Tensor,
    cache: LatentCache,
    sm_scale: float,
    *,
    row_seq: Optional[torch.Tensor] = None,
    kv_len: Optional[torch.Tensor] = None,
    q_rope_pos: Optional[torch.Tensor] = None,
    start_pos: Optional[torch.Tensor] = None,
    rows_per_seq: int = 1,
    rope_abs: bool = False,
    n_splits: int = 1,
    min_chunk: int = 256,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[DecodeWorkspace] = None,
    lse_out: Optional[torch.Tensor] = None,
    merge: bool = True,
    append: Optional[FusedAppend] = None,
    balance: int = 0,
) -> torch.Tensor:
    """Absorbed attention of query rows over the latent cache (+ merge).

    q_abs [rows, H, R_pad] (channels >= the cache's rank are ignored) and
    q_pe [rows, H, P] may be strided views (unit last stride); H is 16, or
    32 for a bf16 model at R_pad <= 256 (one launch of two head groups:
    the cache is streamed once for both).  Addressing:
    explicit (row_seq, kv_len, q_rope_pos) or dense (start_pos [rows /
    rows_per_seq], causal).  Returns o_lat [rows, H, R_pad], whose padding
    channels are 0 (``out`` may be a strided view, e.g. a transpose of a
    [H, rows, R_pad] buffer).  ``lse_out`` [rows, H] fp32, if given, receives
    every row's log-sum-exp (natural log; -inf for an empty row).  With more
    than one split, mla_merge runs after the decode kernel unless
    ``merge`` is False: then rows with several splits leave their partials in
    ``workspace`` for merge_project.  With ``append`` (bf16, dense
    addressing, one row per sequence) the step's new tokens are appended in
    the same launch (mla_decode_attn_append); the result equals append()
    followed by this call.  ``balance`` > 0 asks for a length-balanced
    plan: ``balance`` workgroups share all rows' splits, with one chunk chosen
    on the device from every row's length (see ``balanced_splits``); the
    chunk lands in ``workspace.plan`` for a later merge_project(balanced=True).
    Reference: models/mla.py:417-487 (and :307-323, :409-414 with append).
    """
    cache.validate()
    dev = _need_gpu(q_abs, q_pe, cos_tab, sin_tab, cache.ckv, row_seq, kv_len, q_rope_pos, start_pos)
    dt = cache.model_dtype
    rows = q_abs.shape[0]
    rk, rp = cache.rank, cache.rank_pad
    nh = q_abs.shape[1] if q_abs.dim() == 3 else H
    if nh not in DECODE_HEADS:
        raise ValueError(f"q_abs has {nh} heads; one decode launch takes {DECODE_HEADS}")
    if q_abs.dim() != 3 or tuple(q_abs.shape[1:]) != (nh, rp) or q_abs.stride(2) != 1:
        raise ValueError(f"q_abs must be [rows, {nh}, {rp}] (R_pad) with unit last stride")
    if q_pe.dim() != 3 or tuple(q_pe.shape) != (rows, nh, P) or q_pe.stride(2) != 1:
        raise ValueError(f"q_pe must be [rows, {nh}, {P}] with unit last stride")
    if q_abs.dtype != dt or q_pe.dtype != dt or cos_tab.dtype != dt:
        raise TypeError(f"query and RoPE tensors must be {dt}")
    (p_seq, p_len, p_rope), p_sp = _addressing(
        rows, (row_seq, kv_len, q_rope_pos), start_pos, rows_per_seq, ("row_seq", "kv_len", "q_rope_pos"))
    if out is None:
        out = torch.empty(rows, nh, rp, dtype=dt, device=dev)
    if tuple(out.shape) != (rows, nh, rp) or out.stride(2) != 1 or out.dtype != dt:
        raise ValueError("out must be [rows, H, R_pad] in the model dtype with unit last stride")
    if n_splits > 1:
        if workspace is None:
            workspace = DecodeWorkspace.allocate(rows, n_splits, dev, rank=rk, heads=nh)
        if not workspace.fits(rows, n_splits, rk, nh):
            raise ValueError("workspace does not fit (rows, n_splits, heads, rank)")
    plan = workspace.plan if (balance > 0 and workspace is not None) else None
    lib = _abi.lib()
    stream = _abi.stream_handle(dev)
    if append is not None:
        kv, ln_w, ln_b = append.kv, append.ln_w, append.ln_b
        if start_pos is None or rows_per_seq != 1:
            raise ValueError("a fused append needs dense addressing with one row per sequence")
        if kv.dim() != 2 or kv.shape[0] != rows or kv.shape[1] < rp + P or kv.stride(1) != 1:
            raise ValueError("append.kv must be [rows, >=R_pad+P] with unit last-dim stride")
        if kv.dtype != dt or ln_w.dtype != dt or ln_b.dtype != dt:
            raise TypeError(f"append tensors must be {dt}")
        if not (ln_w.is_contiguous() and ln_b.is_contiguous() and ln_w.numel() in (rk, rp)
                and ln_b.numel() in (rk, rp)):
            raise ValueError("LayerNorm weight / bias must be contiguous [R] or [R_pad]")
        ln_w, ln_b = pad_rank(ln_w.reshape(-1), rk), pad_rank(ln_b.reshape(-1), rk)
        _need_gpu(kv, ln_w, ln_b, append.err_flag)
        _abi.check(
            lib.mla_decode_attn_append(
                kv.data_ptr(), kv.stride(0), ln_w.data_ptr(), ln_b.data_ptr(), float(append.eps),
                _abi.ptr(append.err_flag),
                q_abs.data_ptr(), q_abs.stride(0), q_abs.stride(1),
                q_pe.data_ptr(), q_pe.stride(0), q_pe.stride(1),
                cos_tab.data_ptr(), sin_tab.data_ptr(), cos_tab.shape[0],
                cache.ckv.data_ptr(), cache.kpe.data_ptr(), _abi.ptr(cache.scale),
                cache.ckv.shape[0], cache.ckv.shape[1], p_sp, int(bool(rope_abs)),
                rows, nh, rk, P, float(sm_scale), n_splits, min_chunk, int(balance), _abi.ptr(plan),
                _abi.ptr(workspace.o_part if workspace else None),
                _abi.ptr(workspace.lse_part if workspace else None),
                out.data_ptr(), out.stride(0), out.stride(1), _abi.ptr(lse_out),
                _abi.dtype_code(dt), cache.cache_code, stream,
            )
        )
    else:
        _abi.check(
            lib.mla_decode_attn(
                q_abs.data_ptr(), q_abs.stride(0), q_abs.stride(1),
                q_pe.data_ptr(), q_pe.stride(0), q_pe.stride(1),
                cos_tab.data_ptr(), sin_tab.data_ptr(), cos_tab.shape[0],
                cache.ckv.data_ptr(), cache.kpe.data_ptr(), _abi.ptr(cache.scale),
                cache.ckv.shape[0], cache.ckv.shape[1],
                p_seq, p_len, p_rope, p_sp, int(rows_per_seq), int(bool(rope_abs)),
                rows, nh, rk, P, float(sm_scale), n_splits, min_chunk, int(balance), _abi.ptr(plan),
                _abi.ptr(workspace.o_part if workspace else None),
                _abi.ptr(workspace.lse_part if workspace else None),
                out.data_ptr(), out.stride(0), out.stride(1), _abi.ptr(lse_out),
                _abi.dtype_code(dt), cache.cache_code, stream,
            )
        )
    if n_splits > 1 and merge:
        _abi.check(
            lib.mla_merge(
                workspace.o_part.data_ptr(), workspace.lse_part.data_ptr(), p_seq, p_len, p_sp,
                int(rows_per_seq), cache.ckv.shape[0], cache.ckv.shape[1], rows, nh, rk, n_splits, min_chunk,
                _abi.ptr(plan), out.data_ptr(), out.stride(0), out.stride(1),
                _abi.ptr(lse_out), _abi.dtype_code(dt), stream,
            )
        )
    return out


PREFILL_QUERIES_PER_BLOCK = 8  # mla_prefill_attn: one query per wave, eight waves


def use_prefill(n_seq: int, tokens_per_seq: int, num_cus: int = 256, rank: int = R) -> bool:
    """Whether a dense chunk of ``tokens_per_seq`` tokens per sequence is
    better served by prefill_attention (eight queries share each cache tile)
    than by per-row decode_attention with split-KV: when the chunk alone
    gives about one workgroup per CU (prefill_attention covers ranks up to
    256)."""
    blocks = n_seq * -(-tokens_per_seq // PREFILL_QUERIES_PER_BLOCK)
    return tokens_per_seq >= 8 and blocks >= num_cus and padded_rank(rank) <= 256


def prefill_attention(
    q_abs: torch.Tensor,
    q_pe: torch.Tensor,
    cos_tab: torch.Tensor,
    sin_tab: torch.Tensor,
    cache: LatentCache,
    sm_scale: float,
    *,
    start_pos: torch.Tensor,
    rows_per_seq: int,
    rope_abs: bool = False,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Causal absorbed attention of a prefill chunk (mla_prefill_attn): row r
    is token r % T of sequence r / T and attends to [0, start_pos + r % T + 1).
    Same operands as decode_attention in dense mode; no split-KV; ranks up
    to 256 (use_prefill says when it applies).
    Reference: models/mla.py:417-487 (seqlen > 1)."""
    cache.validate()
    dev = _need_gpu(q_abs, q_pe, cos_tab, sin_tab, cache.ckv, start_pos)
    dt = cache.model_dtype
    rows = q_abs.shape[0]
    rk, rp = cache.rank, cache.rank_pad
    if q_abs.dim() != 3 or tuple(q_abs.shape[1:]) != (H, rp) or q_abs.stride(2) != 1:
        raise ValueError(f"q_abs must be [rows, {H}, {rp}] (R_pad) with unit last stride")
    if q_pe.dim() != 3 or tuple(q_pe.shape) != (rows, H, P) or q_pe.stride(2) != 1:
        raise ValueError(f"q_pe must be [rows, {H}, {P}] with unit last stride")
    if q_abs.dtype != dt or q_pe.dtype != dt or cos_tab.dtype != dt:
        raise TypeError(f"query and RoPE tensors must be {dt}")
    _, p_sp = _addressing(rows, (None, None, None), start_pos, rows_per_seq, ("row_seq", "kv_len", "q_rope_pos"))
    if out is None:
        out = torch.empty(rows, H, rp, dtype=dt, device=dev)
    if tuple(out.shape) != (rows, H, rp) or out.stride(2) != 1 or out.dtype != dt:
        raise ValueError("out must be [rows, H, R_pad] in the model dtype with unit last stride")
    _abi.check(
        _abi.lib().mla_prefill_attn(
            q_abs.data_ptr(), q_abs.stride(0), q_abs.stride(1),
            q_pe.data_ptr(), q_pe.stride(0), q_pe.stride(1),
            cos_tab.data_ptr(), sin_tab.data_ptr(), cos_tab.shape[0],
            cache.ckv.data_ptr(), cache.kpe.data_ptr(), _abi.ptr(cache.scale),
            cache.ckv.shape[0], cache.ckv.shape[1], p_sp, int(rows_per_seq), int(bool(rope_abs)),
            rows, H, rk, P, float(sm_scale),
            out.data_ptr(), out.stride(0), out.stride(1),
            _abi.dtype_code(dt), cache.cache_code, _abi.stream_handle(dev),
        )
    )
    return out


LINEAR_MAX_ROWS = 128


def linear(
    x: torch.Tensor,
    w: torch.Tensor,
    out: Optional[torch.Tensor] = None,
    bias: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """out[b, m, n] = x[b, m, :] . w[b, n, :] (+ bias[b, n]) in bf16 with fp32
    accumulation (mla_linear).  x [batch, M, K], w [batch, N, K], out
    [batch, M, N] and bias [batch, N] may be strided views with a unit last
    stride; 2-D x / w / out (and 1-D bias) are one batch entry.  For the
    decode step's products (M <= 128): wq / wkv_a (models/mla.py:281-288,
    :307), the absorbed W_uk / W_uv products (re-associating :427, :433) and
    wo (:490-495)."""
    squeeze = x.dim() == 2
    if squeeze:
        x, w = x.unsqueeze(0), w.unsqueeze(0)
        out = None if out is None else out.unsqueeze(0)
        bias = None if bias is None else bias.unsqueeze(0)
    dev = _need_gpu(x, w, out, bias)
    if x.dim() != 3 or w.dim() != 3 or x.shape[0] != w.shape[0] or x.shape[2] != w.shape[2]:
        raise ValueError(f"x {tuple(x.shape)} and w {tuple(w.shape)} must be [batch, M, K] / [batch, N, K]")
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise TypeError("linear: bf16 inputs only")
    batch, M, K = x.shape
    N = w.shape[1]
    if out is None:
        out = torch.empty(batch, M, N, dtype=x.dtype, device=dev)
    if tuple(out.shape) != (batch, M, N) or out.dtype != x.dtype:
        raise ValueError(f"out must be [{batch}, {M}, {N}] bf16")
    for t, name in ((x, "x"), (w, "w"), (out, "out")):
        if t.stride(2) != 1:
            raise ValueError(f"{name} needs a unit last stride")
    if bias is not None and (bias.dim() != 2 or tuple(bias.shape) != (batch, N) or bias.stride(1) != 1
                             or bias.dtype != x.dtype):
        raise ValueError(f"bias must be [{batch}, {N}] bf16 with a unit last stride")
    _abi.check(
        _abi.lib().mla_linear(
            x.data_ptr(), x.stride(1), x.stride(0), w.data_ptr(), w.stride(1), w.stride(0),
            _abi.ptr(bias), 0 if bias is None else bias.stride(0),
            out.data_ptr(), out.stride(1), out.stride(0), M, N, K, batch,
            _abi.DTYPE_BF16, _abi.stream_handle(dev),
        )
    )
    return out[0] if squeeze else out


def head_product_ok(K: int, N: int) -> bool:
    """Whether mla_head_product covers a per-head product of this shape."""
    return 64 <= K <= 512 and K % 64 == 0 and N > 0 and N % 4 == 0


def head_product(x: torch.Tensor, w: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[m, h, n] = x[m, h, :] . w[h, n, :] in bf16 with fp32 accumulation
    and one rounding (mla_head_product), for prompt-sized row counts: the
    absorbed products q_nope . W_uk and o_lat . W_uv^T that re-associate the
    einsums of models/mla.py:427 and :433.  x [M, H, K], w [H, N, K] and out
    [M, H, N] may be strided views with a unit last stride (x read in place,
    e.g. the q_nope columns of the wq output)."""
    dev = _need_gpu(x, w, out)
    if x.dim() != 3 or w.dim() != 3 or x.shape[1] != w.shape[0] or x.shape[2] != w.shape[2]:
        raise ValueError(f"x {tuple(x.shape)} and w {tuple(w.shape)} must be [M, H, K] / [H, N, K]")
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise TypeError("head_product: bf16 inputs only")
    M, Hx, K = x.shape
    N = w.shape[1]
    if out is None:
        out = torch.empty(M, Hx, N, dtype=x.dtype, device=dev)
    if tuple(out.shape) != (M, Hx, N) or out.dtype != x.dtype:
        raise ValueError(f"out must be [{M}, {Hx}, {N}] bf16")
    for t, name in ((x, "x"), (w, "w"), (out, "out")):
        if t.stride(2) != 1:
            raise ValueError(f"{name} needs a unit last stride")
    _abi.check(
        _abi.lib().mla_head_product(
            x.data_ptr(), x.stride(0), x.stride(1), w.data_ptr(), w.stride(1), w.stride(0),
            out.data_ptr(), out.stride(0), out.stride(1), M, N, K, Hx,
            _abi.DTYPE_BF16, _abi.stream_handle(dev),
        )
    )
    return out


PACKED_K = (512, 1024, 1536, 2048)


@dataclass
class PackedWeight:
    """A [N, K] bf16 weight in mla_pack_weight's 1 KB-tile layout (flat
    storage of N*K elements)."""

    data: torch.Tensor
    N: int
    K: int


def packed_ok(M: int, N: int, K: int) -> bool:
    """Whether mla_linear_packed covers a product of this shape."""
    return 0 < M <= LINEAR_MAX_ROWS and N > 0 and N % 8 == 0 and K in PACKED_K


def packed_blocks(M: int, N: int, K: int) -> int:
    """Workgroups mla_linear_packed launches for an [M, K] x [N, K]^T product
    (packed_ok shapes).  Mirrors the C++ launcher's grid (launch_linear_packed
    and packed_slab_rows in mla_linear.hip): slabs of 16 / 32 / 64 rows, about
    256 workgroups, at most four 8-row output octets each.  Every workgroup
    takes a CU to itself (its LDS), so a count above the CUs means a second
    round."""
    if K <= 1024 and M > 32:
        ms = 64
    elif K <= 1024 or (K <= 2048 and N // 8 >= 256):
        ms = 32 if M > 16 else 16
    else:
        ms = 16
    slabs = (M + ms - 1) // ms
    n_oct = N // 8
    gx = max((256 + slabs - 1) // slabs, (n_oct + 3) // 4)
    return slabs * min(gx, n_oct)


def pack_weight(w: torch.Tensor) -> PackedWeight:
    """Re-lay a [N, K] bf16 weight (unit last stride) for linear_packed."""
    dev = _need_gpu(w)
    if w.dim() != 2 or w.dtype != torch.bfloat16 or w.stride(1) != 1:
        raise ValueError("pack_weight: w must be a [N, K] bf16 matrix with a unit last stride")
    N, K = w.shape
    out = torch.empty(N * K, dtype=w.dtype, device=dev)
    _abi.check(_abi.lib().mla_pack_weight(w.data_ptr(), w.stride(0), N, K, out.data_ptr(), _abi.DTYPE_BF16,
                                          _abi.stream_handle(dev)))
    return PackedWeight(out, N, K)


def linear_packed(
    x: torch.Tensor,
    wp: PackedWeight,
    out: Optional[torch.Tensor] = None,
    bias: Optional[torch.Tensor] = None,
    advance: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """out[m, n] = x[m, :] . w[n, :] (+ bias[n]) with w packed by pack_weight
    (mla_linear_packed): the decode step's stacked input product and wo
    (models/mla.py:281-288, :307, :490-495).  ``advance`` (a contiguous int32
    device tensor of 1 to 512 entries, not overlapping the operands): the same
    launch adds 1 to each entry (a decode loop's device positions)."""
    dev = _need_gpu(x, wp.data, out, bias, advance)
    if x.dim() != 2 or x.dtype != torch.bfloat16 or x.stride(1) != 1 or x.shape[1] != wp.K:
        raise ValueError(f"x must be [M, {wp.K}] bf16 with a unit last stride")
    M = x.shape[0]
    if out is None:
        out = torch.empty(M, wp.N, dtype=x.dtype, device=dev)
    if tuple(out.shape) != (M, wp.N) or out.dtype != x.dtype or out.stride(1) != 1:
        raise ValueError(f"out must be [{M}, {wp.N}] bf16 with a unit last stride")
    if bias is not None and (bias.dim() != 1 or bias.numel() != wp.N or bias.stride(0) != 1
                             or bias.dtype != x.dtype):
        raise ValueError(f"bias must be a contiguous [{wp.N}] bf16 vector")
    n_adv = 0
    if advance is not None:
        if advance.dtype != torch.int32 or not advance.is_contiguous() or not 1 <= advance.numel() <= 512:
            raise ValueError("advance must be a contiguous int32 tensor of 1 to 512 entries")
        n_adv = advance.numel()
    _abi.check(
        _abi.lib().mla_linear_packed(
            x.data_ptr(), x.stride(0), wp.data.data_ptr(), _abi.ptr(bias), out.data_ptr(), out.stride(0),
            M, wp.N, wp.K, _abi.ptr(advance), n_adv, _abi.DTYPE_BF16, _abi.stream_handle(dev),
        )
    )
    return out


def merge_project(
    o_lat: torch.Tensor,
    w_uv: torch.Tensor,
    out: torch.Tensor,
    cache: LatentCache,
    *,
    n_splits: int,
    min_chunk: int,
    workspace: Optional[DecodeWorkspace] = None,
    row_seq: Optional[torch.Tensor] = None,
    kv_len: Optional[torch.Tensor] = None,
    start_pos: Optional[torch.Tensor] = None,
    rows_per_seq: int = 1,
    balanced: bool = False,
) -> torch.Tensor:
    """out[r, h, :] = W_uv[h] . o_lat[r, h, :] where o_lat is merged from the
    split partials left by ``decode_attention(..., merge=False)`` (or read
    from ``o_lat`` for single-split rows); mla_merge_project.  o_lat and w_uv
    [H, Dv, R_pad] hold R_pad channels (w_uv a view of wkv_b.weight when R =
    R_pad, else a zero-padded copy); out [rows, H, Dv] may be a view of wo's
    [rows, H*Dv] input.  Addressing and split plan must be the ones the
    decode call used (``balanced``: the decode call had ``balance`` > 0 and
    left its chunk in ``workspace.plan``).  Reference: models/mla.py:433,
    :490-491."""
    dev = _need_gpu(o_lat, w_uv, out, row_seq, kv_len, start_pos)
    rows = o_lat.shape[0]
    Dv = w_uv.shape[1]
    rk, rp = cache.rank, cache.rank_pad
    nh = o_lat.shape[1] if o_lat.dim() == 3 else H
    if nh not in DECODE_HEADS:
        raise ValueError(f"o_lat has {nh} heads; merge_project takes {DECODE_HEADS}")
    if o_lat.dim() != 3 or tuple(o_lat.shape[1:]) != (nh, rp) or o_lat.stride(2) != 1:
        raise ValueError(f"o_lat must be [rows, {nh}, {rp}] (R_pad) with unit last stride")
    if w_uv.dim() != 3 or tuple(w_uv.shape) != (nh, Dv, rp) or w_uv.stride(2) != 1:
        raise ValueError(f"w_uv must be [{nh}, Dv, {rp}] (R_pad) with unit last stride")
    if tuple(out.shape) != (rows, nh, Dv) or out.stride(2) != 1:
        raise ValueError(f"out must be [{rows}, {nh}, {Dv}] with unit last stride")
    if not (o_lat.dtype == w_uv.dtype == out.dtype == torch.bfloat16):
        raise TypeError("merge_project: bf16 tensors only")
    (p_seq, p_len, _), p_sp = _addressing(
        rows, (row_seq, kv_len, None), start_pos, rows_per_seq, ("row_seq", "kv_len", "q_rope_pos"))
    if (n_splits > 1 or balanced) and (workspace is None or not workspace.fits(rows, n_splits, rk, nh)):
        raise ValueError("merge_project needs the decode call's workspace")
    _abi.check(
        _abi.lib().mla_merge_project(
            _abi.ptr(workspace.o_part if n_splits > 1 else None),
            _abi.ptr(workspace.lse_part if n_splits > 1 else None),
            o_lat.data_ptr(), o_lat.stride(0), o_lat.stride(1),
            p_len, p_seq, p_sp, int(rows_per_seq), cache.ckv.shape[0], cache.ckv.shape[1],
            rows, nh, rk, n_splits, min_chunk, _abi.ptr(workspace.plan if balanced else None),
            w_uv.data_ptr(), w_uv.stride(1), w_uv.stride(0), Dv,
            out.data_ptr(), out.stride(0), out.stride(1), _abi.DTYPE_BF16, _abi.stream_handle(dev),
        )
    )
    return out
