"""Per-kernel oracles in numpy / fp64 (TEST INFRASTRUCTURE ONLY).

Each function states what one HIP kernel must produce and how the statement
itself is pinned (closed forms, library routines, brute force) by the tests
in tests/test_oracle.py.
"""
from __future__ import annotations

import math

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


def f64_to_bf16_bits(d: np.ndarray) -> np.ndarray:
    """One rounding fp64 -> bf16 (round-to-odd to fp32, then RNE to bf16).
    Pinned against exact rational rounding (fractions) on random samples."""
    d = np.asarray(d, dtype=np.float64)
    f = d.astype(np.float32)
    inexact = (f.astype(np.float64) != d) & np.isfinite(d)
    u = f.view(np.uint32).copy()
    away = np.abs(f.astype(np.float64)) > np.abs(d)
    u = np.where(inexact & away, u - 1, u)
    u = np.where(inexact, u | 1, u)
    return f32_to_bf16_bits(u.view(np.float32))


def f32_to_e4m3_codes(x: np.ndarray) -> np.ndarray:
    """fp32 -> e4m3fn codes through torch's own cast (RNE, NaN at >= 464)."""
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return t.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def e4m3_codes_to_f32(c: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(c, dtype=np.uint8))
    return t.view(torch.float8_e4m3fn).to(torch.float32).numpy()


# ---------------------------------------------------------------- LayerNorm
def _butterfly(s: np.ndarray) -> np.ndarray:
    """xor-butterfly over the 64 lanes of the last axis, distances 1..32."""
    lanes = np.arange(64)
    for m in (1, 2, 4, 8, 16, 32):
        s = s + s[..., lanes ^ m]
    return s


def layernorm_f64(c: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float) -> np.ndarray:
    """kv_norm (mla.py:107, :409) in fp64 with the append kernel's reduction
    order, for any rank R = c.shape[-1] up to 512: the row is padded with
    zeros to R_pad = 64 * ceil(R / 64), lane l holds channels K*l .. K*l+K-1
    (K = R_pad / 64) summed left to right (padding adds +0.0), then an xor
    butterfly, times fl64(1 / R); the variance sums only the R real channels.
    Returns unrounded fp64 y [N, R].  ``eps`` is used as its fp32 value, as
    torch's LayerNorm does.  Pinned against torch.nn.functional.layer_norm in
    fp64 (agreement ~1e-15) and the mean-0 / var-1 invariants; for R = 256
    the order is lane l holding channels 4l..4l+3."""
    x0 = np.asarray(c, dtype=np.float64)
    Rr = x0.shape[-1]
    K = -(-Rr // 64)
    rp = 64 * K
    x = np.zeros(x0.shape[:-1] + (rp,), dtype=np.float64)
    x[..., :Rr] = x0
    x = x.reshape(-1, 64, K)
    valid = (np.arange(rp) < Rr).reshape(64, K)
    s = x[..., 0].copy()
    for i in range(1, K):
        s = s + x[..., i]
    inv_r = 1.0 / float(Rr)  # fp64, as the kernels receive it
    mean = _butterfly(s)[..., :1] * inv_r  # [N, 1]
    d = np.where(valid, x - mean[..., None], 0.0)
    q = d[..., 0] * d[..., 0]
    for i in range(1, K):
        q = q + d[..., i] * d[..., i]
    var = _butterfly(q)[..., :1] * inv_r
    rstd = 1.0 / np.sqrt(var + float(np.float32(eps)))
    wp = np.zeros(rp, np.float64)
    bp = np.zeros(rp, np.float64)
    wp[:Rr] = np.asarray(w, np.float64).reshape(-1)
    bp[:Rr] = np.asarray(b, np.float64).reshape(-1)
    y = np.where(valid, (d * rstd[..., None]) * wp.reshape(64, K) + bp.reshape(64, K), 0.0)
    return y.reshape(-1, rp)[:, :Rr]


def layernorm_exact(c, w, b, eps: float, dtype: torch.dtype) -> torch.Tensor:
    """Exactly-rounded LayerNorm output in ``dtype`` (what the cache holds)."""
    y = layernorm_f64(c, w, b, eps)
    if dtype == torch.bfloat16:
        return torch.from_numpy(f64_to_bf16_bits(y).view(np.int16)).view(torch.bfloat16)
    if dtype == torch.float32:
        return torch.from_numpy(y.astype(np.float32))
    raise TypeError(dtype)


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
