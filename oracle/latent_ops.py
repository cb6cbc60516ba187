"""Per-kernel oracles in numpy / fp64 (TEST INFRASTRUCTURE ONLY).

Each function states what one HIP kernel must produce and how the statement
itself is pinned (closed forms, library routines, brute force) by the tests
in tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np
import torch

R, P, H = 256, 64, 16


# ----------------------------------------------------------------- rounding
def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """RNE fp32 -> bf16 bits (eager PyTorch's cast).  Pinned against
    ``torch.Tensor.to(torch.bfloat16)`` on random and edge-case values."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, 0x7FC0, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_e4m3_codes(x: np.ndarray) -> np.ndarray:
    """fp32 -> e4m3fn codes through torch's own cast (RNE, NaN at >= 464)."""
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return t.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def e4m3_codes_to_f32(c: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(c, dtype=np.uint8))
    return t.view(torch.float8_e4m3fn).to(torch.float32).numpy()


# ---------------------------------------------------------------- LayerNorm
_HERE = os.path.dirname(os.path.abspath(__file__))
ATEN_LN_SRC = os.path.join(_HERE, "aten_layernorm.c")
ATEN_LN_LIB = os.path.join(_HERE, "libaten_layernorm.so")
_aten_ln = None


def build_aten_layernorm(force: bool = False) -> str:
    """Compile oracle/aten_layernorm.c (gcc, contraction off: every fused
    multiply-add of the statement is an explicit fmaf) next to its source."""
    if force or not os.path.exists(ATEN_LN_LIB) or os.path.getmtime(ATEN_LN_LIB) < os.path.getmtime(ATEN_LN_SRC):
        tmp = ATEN_LN_LIB + f".tmp{os.getpid()}"
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-shared", "-fPIC", ATEN_LN_SRC,
                        "-o", tmp, "-lm"], check=True, capture_output=True, text=True)
        os.replace(tmp, ATEN_LN_LIB)
    return ATEN_LN_LIB


def _aten_ln_lib():
    global _aten_ln
    if _aten_ln is None:
        lib = ctypes.CDLL(build_aten_layernorm())
        vp, i64, i32, f = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        for name in ("aten_layernorm_bf16", "aten_layernorm_f32"):
            fn = getattr(lib, name)
            fn.argtypes = [vp, i64, i32, i32, vp, vp, f, vp, i64, vp, vp, i32]
            fn.restype = None
        _aten_ln = lib
    return _aten_ln


def layernorm_aten(c: torch.Tensor, w: torch.Tensor, b: torch.Tensor, eps: float, variant: int = 0):
    """kv_norm (mla.py:107, :409) as PyTorch's CPU LayerNorm computes it, op
    for op (oracle/aten_layernorm.c): c [M, N] bf16 or fp32 rows, w / b [N] in
    the same dtype.  Returns (y [M, N] in c's dtype, mean [M], rstd [M] fp32).
    ``variant`` plants single-site mistakes for the tests that pin it.
    Pinned bit for bit against torch.nn.functional.layer_norm /
    torch.native_layer_norm on CPU (tests/test_oracle.py)."""
    lib = _aten_ln_lib()
    c = c.detach().cpu().contiguous()
    M, N = c.shape
    w = w.detach().cpu().to(c.dtype).contiguous()
    b = b.detach().cpu().to(c.dtype).contiguous()
    y = torch.empty_like(c)
    mean = torch.empty(M, dtype=torch.float32)
    rstd = torch.empty(M, dtype=torch.float32)
    fn = {torch.bfloat16: lib.aten_layernorm_bf16, torch.float32: lib.aten_layernorm_f32}[c.dtype]
    fn(c.data_ptr(), N, M, N, w.data_ptr(), b.data_ptr(), float(np.float32(eps)), y.data_ptr(), N,
       mean.data_ptr(), rstd.data_ptr(), int(variant))
    return y, mean, rstd


def fp8_quantize(y: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token e4m3 encode of the bf16 latent rows y [N, R] (torch emulation):
    scale = max(amax, 1e-12) / 448 in fp32, codes = RNE(y / scale)."""
    yf = y.float()
    amax = yf.abs().amax(dim=-1)
    scale = torch.clamp(amax, min=1e-12) / 448.0
    codes = (yf / scale[:, None]).to(torch.float8_e4m3fn).view(torch.uint8)
    return codes, scale


def fp8_dequantize(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    return codes.view(torch.float8_e4m3fn).float() * scale[..., None]


# --------------------------------------------------------------------- RoPE
def rope_interleaved(x: torch.Tensor, cos_half: torch.Tensor, sin_half: torch.Tensor) -> torch.Tensor:
    """Per-op-rounded interleaved RoPE in x's dtype (positional_encoding.py:
    37-41, :57-60).  x [..., P], cos/sin [..., P/2] broadcastable."""
    x1, x2 = x[..., 0::2], x[..., 1::2]
    o1 = x1 * cos_half - x2 * sin_half
    o2 = x2 * cos_half + x1 * sin_half
    return torch.stack([o1, o2], dim=-1).flatten(-2)


# ---------------------------------------------------------------- attention
def split_chunk(L: int, n_splits: int, min_chunk: int) -> int:
    c = max(min_chunk, -(-L // n_splits))
    return (c + 15) // 16 * 16


def split_count(L: int, n_splits: int, min_chunk: int) -> int:
    if L <= 0:
        return 0
    c = split_chunk(L, n_splits, min_chunk)
    return -(-L // c)


def absorbed_attention_f64(q_abs, q_pe_rot, ckv, kpe, kv_len, row_seq, scale, ckv_scale=None):
    """o_lat[r, h] = sum_t softmax_t(scale * (q_abs.c_t + q_pe.k_pe_t)) c_t in
    fp64 (the decode kernel's maths, re-associated from mla.py:427-437).
    Inputs are torch tensors; ckv may be e4m3 codes with ckv_scale.
    Returns (o_lat [rows, H, R], lse [rows, H]) as float64.
    Pinned by tests: equals the un-absorbed reference formulation in fp64."""
    qa = q_abs.double()
    qp = q_pe_rot.double()
    if ckv.dtype == torch.uint8:
        c_all = fp8_dequantize(ckv, ckv_scale).double()
    else:
        c_all = ckv.double()
    p_all = kpe.double()
    rows = qa.shape[0]
    o = torch.zeros(rows, qa.shape[1], c_all.shape[-1], dtype=torch.float64)
    lse = torch.full((rows, qa.shape[1]), -math.inf, dtype=torch.float64)
    for r in range(rows):
        L = int(kv_len[r])
        if L <= 0:
            continue
        b = int(row_seq[r])
        c = c_all[b, :L]
        s = (qa[r] @ c.T + qp[r] @ p_all[b, :L].T) * scale  # [H, L]
        lse[r] = torch.logsumexp(s, dim=-1)
        o[r] = torch.softmax(s, dim=-1) @ c
    return o, lse


def merge_partials_f64(o_parts: torch.Tensor, lses: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Log-sum-exp merge: o_parts [S, ..., R], lses [S, ...] -> (o, lse)."""
    lses = lses.double()
    m = lses.max(dim=0).values
    w = torch.exp(lses - m)
    w = torch.where(torch.isfinite(lses), w, torch.zeros_like(w))
    tot = w.sum(dim=0)
    o = (w[..., None] * o_parts.double()).sum(dim=0) / tot[..., None]
    return o, m + torch.log(tot)
