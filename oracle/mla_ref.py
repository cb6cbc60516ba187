"""Op-for-op CPU restatement of the reference MLA absorb branch (oracle).

Follows Orolol/swamla models/mla.py and models/positional_encoding.py line by
line, including their quirks:
  * RoPE positions are 0..T-1 of the current call whatever ``start_pos`` is
    (positional_encoding.py:30-34, :49-50; mla.py:299-303, :318-323);
  * interleaved pairs, cos/sin buffers converted with the module dtype and
    every op rounded in that dtype (positional_encoding.py:21-28, :57-60);
  * a call longer than the table rebuilds it in fp32 on the buffers' device
    (positional_encoding.py:44-46, :64-86), so a bf16 module's rotation turns
    fp32 and its SDPA then receives fp32 queries/keys with bf16 values;
  * caches are ``torch.zeros`` buffers created by ``set_inference_mode``
    (mla.py:207-215), so they must be enabled before ``.to(dtype)``;
  * attention re-projects the whole cache through wkv_b and runs SDPA with
    ``is_causal = mask is None and seqlen > 1`` (mla.py:402-487);
  * ``softmax_scale = qk_head_dim ** -0.5`` (mla.py:118).
Pinned by tests/golden (fixtures written by importing the real reference in
the build container, tests/golden/make_golden.py): outputs and caches must
match bit-exactly.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass
class MLAConfig:
    """The attributes the reference MLA reads (mla.py:75-170)."""

    n_embd: int = 1024
    n_head: int = 16
    q_lora_rank: int = 0
    kv_lora_rank: int = 256
    qk_nope_head_dim: int = 128
    qk_rope_head_dim: int = 64
    v_head_dim: int = 128
    max_batch_size: int = 8
    max_seq_len: int = 4096
    dropout: float = 0.0
    bias: bool = False
    attn_impl: str = "absorb"


class RefRoPE(nn.Module):
    """positional_encoding.py:9-91 (table, interleaved rotation, forward)."""

    def __init__(self, dim: int, max_seq_len: int = 2048, base: int = 10000):
        super().__init__()
        self.dim = dim
        self.max_seq_len = max_seq_len
        self.base = base
        inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))  # :21
        t = torch.arange(max_seq_len).type_as(inv_freq)
        freqs = torch.einsum("i,j->ij", t, inv_freq)
        emb = torch.cat((freqs, freqs), dim=-1)
        self.register_buffer("cos_cached", emb.cos().view(1, 1, max_seq_len, dim), persistent=False)
        self.register_buffer("sin_cached", emb.sin().view(1, 1, max_seq_len, dim), persistent=False)

    def _rotate_half(self, x: torch.Tensor, seq_len: int) -> torch.Tensor:  # :30-62
        B, Hh, T, D = x.shape
        x = x.contiguous()
        xr = x.view(B, Hh, T, D // 2, 2)
        x1, x2 = xr[..., 0].contiguous(), xr[..., 1].contiguous()
        if T > self.max_seq_len:
            self._extend_cos_sin_cache(T)
        cos = self.cos_cached[:, :, :T, : (D // 2)].expand(B, Hh, T, -1).contiguous()
        sin = self.sin_cached[:, :, :T, : (D // 2)].expand(B, Hh, T, -1).contiguous()
        rotated = torch.stack([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)
        return rotated.view(B, Hh, T, D).contiguous()

    def _extend_cos_sin_cache(self, new_max_len: int) -> None:  # :64-86
        """Rebuilds the table in fp32 on the buffers' device for new_max_len
        positions and replaces the buffers (their dtype becomes fp32)."""
        if new_max_len <= self.max_seq_len:
            return
        self.max_seq_len = new_max_len
        dev = self.cos_cached.device
        inv_freq = (1.0 / (self.base ** (torch.arange(0, self.dim, 2).float() / self.dim))).to(dev)
        t = torch.arange(new_max_len, device=dev).type_as(inv_freq)
        emb = torch.cat((torch.einsum("i,j->ij", t, inv_freq),) * 2, dim=-1)
        self.register_buffer("cos_cached", emb.cos().view(1, 1, new_max_len, self.dim), persistent=False)
        self.register_buffer("sin_cached", emb.sin().view(1, 1, new_max_len, self.dim), persistent=False)

    def forward(self, x: torch.Tensor, seq_len=None) -> torch.Tensor:  # :88-91
        if seq_len is None:
            seq_len = x.shape[-2]
        return self._rotate_half(x, seq_len)


class RefMLA(nn.Module):
    """mla.py:53-495, absorb branch only, SDPA backend (cuDNN is off: qk 192 > 128).

    ``fp8_cache=True`` is the PyTorch emulation of the e4m3 latent cache (no
    reference counterpart): each appended latent row is quantised per token
    (latent_ops.fp8_quantize) and attention reads the dequantised rows,
    rounded to the model dtype."""

    def __init__(self, config, fp8_cache: bool = False):
        super().__init__()
        self.fp8_cache = fp8_cache
        self.dim = config.n_embd
        self.n_heads = config.n_head
        self.q_lora_rank = config.q_lora_rank
        self.kv_lora_rank = config.kv_lora_rank
        self.qk_nope_head_dim = config.qk_nope_head_dim
        self.qk_rope_head_dim = config.qk_rope_head_dim
        self.qk_head_dim = self.qk_nope_head_dim + self.qk_rope_head_dim
        self.v_head_dim = config.v_head_dim
        bias = config.bias
        if self.q_lora_rank == 0:
            self.wq = nn.Linear(self.dim, self.n_heads * self.qk_head_dim, bias=bias)
        else:
            self.wq_a = nn.Linear(self.dim, self.q_lora_rank, bias=bias)
            self.q_norm = nn.LayerNorm(self.q_lora_rank)
            self.wq_b = nn.Linear(self.q_lora_rank, self.n_heads * self.qk_head_dim, bias=bias)
        self.wkv_a = nn.Linear(self.dim, self.kv_lora_rank + self.qk_rope_head_dim, bias=bias)
        self.kv_norm = nn.LayerNorm(self.kv_lora_rank)
        self.wkv_b = nn.Linear(self.kv_lora_rank, self.n_heads * (self.qk_nope_head_dim + self.v_head_dim), bias=bias)
        self.wo = nn.Linear(self.n_heads * self.v_head_dim, self.dim, bias=bias)
        self.softmax_scale = self.qk_head_dim ** -0.5
        self.max_batch_size = config.max_batch_size
        self.max_seq_len = config.max_seq_len
        self.rope = RefRoPE(self.qk_rope_head_dim, self.max_seq_len)
        self.inference_mode = False
        self.kv_cache = None
        self.pe_cache = None

    def set_inference_mode(self, mode: bool = True) -> None:  # mla.py:184-225
        """As in the reference: raises KeyError while ``kv_cache``/``pe_cache``
        are still the plain ``None`` attributes set by __init__ (mla.py:180-182
        vs register_buffer at :209); drive it through ``enable_cache``."""
        if mode == self.inference_mode:
            return
        self.inference_mode = mode
        if mode:
            self.register_buffer(
                "kv_cache", torch.zeros(self.max_batch_size, self.max_seq_len, self.kv_lora_rank), persistent=False
            )
            self.register_buffer(
                "pe_cache", torch.zeros(self.max_batch_size, self.max_seq_len, self.qk_rope_head_dim), persistent=False
            )
        else:
            for name in ("kv_cache", "pe_cache"):
                if hasattr(self, name):
                    delattr(self, name)

    def project(self, x: torch.Tensor):
        """mla.py:277-323: q_nope, RoPE'd q_pe, raw c (split view), RoPE'd k_pe."""
        bsz, seqlen, _ = x.size()
        q = self.wq(x) if self.q_lora_rank == 0 else self.wq_b(self.q_norm(self.wq_a(x)))
        q = q.view(bsz, seqlen, self.n_heads, self.qk_head_dim)
        q_nope, q_pe = torch.split(q, [self.qk_nope_head_dim, self.qk_rope_head_dim], dim=-1)
        q_pe = q_pe.transpose(1, 2).contiguous()
        q_pe = self.rope(q_pe)
        q_pe = q_pe.transpose(1, 2).contiguous()
        kv, k_pe = self.project_kv(x)
        return q_nope, q_pe, kv, k_pe

    def project_kv(self, x: torch.Tensor):
        """mla.py:307-323: raw c (split view) and RoPE'd k_pe."""
        bsz, seqlen, _ = x.size()
        kv = self.wkv_a(x)
        kv, k_pe = torch.split(kv, [self.kv_lora_rank, self.qk_rope_head_dim], dim=-1)
        k_pe = k_pe.view(bsz, seqlen, 1, -1).transpose(1, 2)
        k_pe = self.rope(k_pe.contiguous()).squeeze(1)
        return kv, k_pe

    def cache_rows(self, kv: torch.Tensor) -> torch.Tensor:
        """mla.py:409 (kv_norm), plus the e4m3 round trip of the emulated
        fp8 cache."""
        kv_norm_tensor = self.kv_norm(kv)
        if self.fp8_cache:
            from .latent_ops import fp8_dequantize, fp8_quantize

            codes, scale = fp8_quantize(kv_norm_tensor.reshape(-1, self.kv_lora_rank))
            kv_norm_tensor = fp8_dequantize(codes, scale).to(kv.dtype).view_as(kv_norm_tensor)
        return kv_norm_tensor

    def fill_cache(self, x: torch.Tensor, start_pos: int) -> None:
        """The cache writes of forward (mla.py:307-323, :409-414) without the
        query projection or attention: what a prompt pass leaves in
        kv_cache / pe_cache."""
        bsz, seqlen, _ = x.size()
        kv, k_pe = self.project_kv(x)
        self.kv_cache[:bsz, start_pos:start_pos + seqlen] = self.cache_rows(kv)
        self.pe_cache[:bsz, start_pos:start_pos + seqlen] = k_pe

    def forward(self, x: torch.Tensor, start_pos: int, freqs_cis=None, mask=None) -> torch.Tensor:
        """``mask``: additive [S, T] mask, expanded and cast to the query
        dtype as mla.py:473-478 does (is_causal is then off, :483)."""
        bsz, seqlen, _ = x.size()
        end_pos = start_pos + seqlen
        q_nope, q_pe, kv, k_pe = self.project(x)
        wkv_b = self.wkv_b.weight.view(self.n_heads, -1, self.kv_lora_rank)  # :404-406
        kv_norm_tensor = self.cache_rows(kv)  # :409
        if self.inference_mode:
            self.kv_cache[:bsz, start_pos:end_pos] = kv_norm_tensor  # :413-414
            self.pe_cache[:bsz, start_pos:end_pos] = k_pe
            kv_to_use = self.kv_cache[:bsz, :end_pos]
            pe_to_use = self.pe_cache[:bsz, :end_pos]
        else:
            kv_to_use, pe_to_use = kv_norm_tensor, k_pe
        v = torch.einsum("btc,hdc->bthd", kv_to_use, wkv_b[:, -self.v_head_dim:])  # :427
        q_full = torch.cat([q_nope, q_pe], dim=-1)
        k_nope_full = torch.einsum("btc,hdc->bthd", kv_to_use, wkv_b[:, : self.qk_nope_head_dim])  # :433
        pe_expanded = pe_to_use.unsqueeze(2).expand(-1, -1, self.n_heads, -1)
        k_full = torch.cat([k_nope_full, pe_expanded], dim=-1)
        q_sdpa = q_full.transpose(1, 2).contiguous()  # :466-468
        k_sdpa = k_full.transpose(1, 2).contiguous()
        v_sdpa = v.transpose(1, 2).contiguous()
        attn_mask = None
        if mask is not None:  # :474-478
            attn_mask = mask.unsqueeze(0).unsqueeze(0).expand(bsz, self.n_heads, -1, -1).to(q_sdpa.dtype)
        attn = F.scaled_dot_product_attention(  # :581-595 (no cuDNN, dropout 0 in eval)
            q_sdpa, k_sdpa, v_sdpa, attn_mask=attn_mask, dropout_p=0.0,
            is_causal=mask is None and seqlen > 1, scale=self.softmax_scale,
        )
        x = attn.transpose(1, 2).contiguous().reshape(bsz, seqlen, -1)
        return self.wo(x)


def enable_cache(module: nn.Module) -> None:
    """Harness step that makes the reference's cache reachable: drop the plain
    ``None`` attributes __init__ assigns (mla.py:177-182), then
    ``set_inference_mode(True)``.  Call before ``.to(dtype)`` (mla.py:207-215
    allocates fp32 on the default device)."""
    for name in ("k_cache", "v_cache", "kv_cache", "pe_cache"):
        if name in module.__dict__:
            del module.__dict__[name]
    module.set_inference_mode(True)


def init_weights(module: nn.Module, seed: int, ln_random: bool = False) -> None:
    """N(0, 0.02) Linear weights drawn from a CPU generator in parameter order
    (swa_mla_model.py:314-320 initialises Linears this way and leaves
    LayerNorm at weight 1 / bias 0).  ``ln_random`` also randomises kv_norm
    (w ~ 1 + N(0, 0.1), b ~ N(0, 0.1)) so tests exercise the affine terms."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in module.named_parameters():
            if name.startswith(("wq", "wkv_a", "wkv_b", "wo")) and name.endswith("weight"):
                p.copy_(torch.randn(p.shape, generator=g) * 0.02)
            elif name.endswith("bias") and not name.startswith(("kv_norm", "q_norm")):
                p.zero_()
        if ln_random:
            module.kv_norm.weight.copy_(1.0 + 0.1 * torch.randn(module.kv_norm.weight.shape, generator=g))
            module.kv_norm.bias.copy_(0.1 * torch.randn(module.kv_norm.bias.shape, generator=g))
