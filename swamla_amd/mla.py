"""Drop-in ``MLA`` module whose inference path runs on the MI355X kernels.

Reference: models/mla.py:53-693 (Orolol/swamla).  Constructor, attribute and
parameter names (``wq`` | ``wq_a``/``q_norm``/``wq_b``, ``wkv_a``,
``kv_norm``, ``wkv_b``, ``wo``), ``forward(x, start_pos, ...)``,
``set_inference_mode`` and ``clear_cache`` follow the reference so state
dicts load unchanged and callers need no edits.

What runs where (per forward, bf16 model):
  decode-sized calls (<= 128 query rows, the one-token step):
    mla_linear_packed  x . [W_uk^T wq_nope | wq_pe | wkv_a]^T (q_abs, q_pe, kv)
                       (the library GEMM when its grid would need a second
                       round of workgroups, e.g. 128 rows)
    mla_decode_attn_append  append (kv_norm + RoPE(k_pe) + e4m3 + scatter)
                       folded into the split-KV attention launch (T = 1;
                       longer chunks run mla_append first)
    mla_merge_project  split merge + o = o_lat . W_uv^T in wo's layout
    mla_linear_packed  wo
  prompt-sized calls:
    ATen GEMMs         wq / wkv_a / wo
    mla_head_product   q_abs = q_nope . W_uk and o = o_lat . W_uv^T
    mla_append, then mla_prefill_attn (or mla_decode_attn + mla_merge)
  fp32 models use the ATen products and batched absorption around mla_append
  and the fp32 decode kernel.  The attention launches take 16 heads each,
  and a bf16 decode launch over a bf16 cache of R_pad <= 256 also 32 (two head
  groups in one workgroup, the cache streamed once for both): other head
  counts run as ceil(H / 16) launches over zero-padded query heads (the fused
  decode step is built for 16 and 32 heads).

Differences from the reference, all deliberate:
  * attention is absorbed: the reference re-projects the whole cache through
    wkv_b every step (mla.py:427-437); here the query is projected into the
    latent space instead (same maths, re-associated, bf16 tolerance);
  * ``start_pos`` may also be an int tensor [B] (per-sequence positions,
    ragged batches); the reference takes one int for the whole batch;
  * chunked prefill (T > 1 at start_pos > 0) is causal bottom-right; the
    reference's SDPA ``is_causal`` is top-left there (mla.py:483);
  * caches are allocated in the module's dtype and device (the reference
    allocates fp32 on the default device, mla.py:207-215);
  * ``cache_dtype="fp8_e4m3"`` stores the latent as e4m3fn codes with one
    fp32 scale per token (``kv_scale``);
  * ``kv_cache`` holds R_pad = 64 * ceil(kv_lora_rank / 64) channels per
    token, channels kv_lora_rank.. zero (the kernels' row layout; the same
    shape as the reference's whenever kv_lora_rank is a multiple of 64);
  * ``clear_cache()`` also leaves inference mode, so the next
    ``set_inference_mode(True)`` reallocates (the reference leaves None
    caches behind and its next forward fails);
  * ``mask``: the additive causal mask SWAMLAModel builds for a prompt at
    start_pos 0 is accepted (it equals the causal attention the kernels
    run); any other mask raises ``NotImplementedError``;
  * positions outside the cache raise: at once when known on the host (int
    or CPU tensor ``start_pos``), else from the kernels' error flag at the
    next eager call or ``check_cache_errors()``;
  * the training / autograd path, ``position_ids`` and ``cu_seqlens``
    backends and ``attn_impl="naive"`` are not part of this path and raise
    ``NotImplementedError``.
"""
from __future__ import annotations

import math
from typing import Optional, Union

import torch
import torch.nn as nn

from . import kernels
from .kernels import DecodeWorkspace, LatentCache
from .rope import RoPE

RopeMode = str  # "chunk" (reference: positions 0..T-1 of the call) or "absolute"


class MLA(nn.Module):
    def __init__(self, config, cache_dtype: Optional[str] = None, rope_positions: Optional[str] = None):
        super().__init__()
        # --- mla.py:73-118: dimensions, projections, scale
        self.dim = config.n_embd if hasattr(config, "n_embd") else config.dim
        self.n_heads = config.n_head if hasattr(config, "n_head") else config.n_heads
        self.world_size = getattr(config, "world_size", 1)
        self.n_local_heads = self.n_heads // self.world_size
        self.q_lora_rank = getattr(config, "q_lora_rank", 0)
        self.kv_lora_rank = getattr(config, "kv_lora_rank", 512)
        self.qk_nope_head_dim = getattr(config, "qk_nope_head_dim", 128)
        self.qk_rope_head_dim = getattr(config, "qk_rope_head_dim", 64)
        self.qk_head_dim = self.qk_nope_head_dim + self.qk_rope_head_dim
        self.v_head_dim = getattr(config, "v_head_dim", 128)
        self.dropout = getattr(config, "dropout", 0.0)
        bias = config.bias if hasattr(config, "bias") else False

        if self.q_lora_rank == 0:
            self.wq = nn.Linear(self.dim, self.n_heads * self.qk_head_dim, bias=bias)
        else:
            self.wq_a = nn.Linear(self.dim, self.q_lora_rank, bias=bias)
            self.q_norm = nn.LayerNorm(self.q_lora_rank)
            self.wq_b = nn.Linear(self.q_lora_rank, self.n_heads * self.qk_head_dim, bias=bias)
        self.wkv_a = nn.Linear(self.dim, self.kv_lora_rank + self.qk_rope_head_dim, bias=bias)
        self.kv_norm = nn.LayerNorm(self.kv_lora_rank)
        self.wkv_b = nn.Linear(
            self.kv_lora_rank, self.n_heads * (self.qk_nope_head_dim + self.v_head_dim), bias=bias
        )
        self.wo = nn.Linear(self.n_heads * self.v_head_dim, self.dim, bias=bias)
        self.attn_dropout = nn.Dropout(self.dropout)
        self.resid_dropout = nn.Dropout(self.dropout)

        self.softmax_scale = self.qk_head_dim ** -0.5
        rope_factor = getattr(config, "rope_factor", 1.0)
        if rope_factor > 1.0 and hasattr(config, "original_seq_len") and hasattr(config, "max_seq_len"):
            if config.max_seq_len > config.original_seq_len:  # mla.py:121-126
                mscale = getattr(config, "mscale", 1.0)
                mscale = 0.1 * mscale * math.log(rope_factor) + 1.0
                self.softmax_scale = self.softmax_scale * mscale * mscale

        # --- mla.py:130-132, :172: cache geometry and RoPE (base 10000)
        self.max_batch_size = getattr(config, "max_batch_size", 8)
        self.max_seq_len = getattr(config, "max_seq_len", 4096)
        self.attn_impl = getattr(config, "attn_impl", "absorb")
        self.rope = RoPE(self.qk_rope_head_dim, self.max_seq_len)

        self.cache_dtype = cache_dtype if cache_dtype is not None else getattr(config, "kv_cache_dtype", None)
        if self.cache_dtype not in (None, "model", "fp8_e4m3"):
            raise ValueError(f"cache_dtype must be None/'model' or 'fp8_e4m3', got {self.cache_dtype!r}")
        self.rope_positions: RopeMode = rope_positions or getattr(config, "rope_positions", "chunk")
        if self.rope_positions not in ("chunk", "absolute"):
            raise ValueError("rope_positions must be 'chunk' or 'absolute'")

        self.inference_mode = False
        self.k_cache = None
        self.v_cache = None
        self.kv_cache = None
        self.pe_cache = None
        self.kv_scale = None
        self._absorbed = None  # (key, W_uk [H,nope,R], W_uv^T [H,R,v])
        self._decode_w = None  # (key, stacked absorbed-query / q_pe / wkv_a weight, stacked bias, packed)
        self._wo_packed = None  # (key, wo.weight packed for mla_linear_packed)
        self._padded_w = {}  # name -> (key, zero-padded copy to R_pad): kv_norm, wkv_a, W_uv
        self._workspace: Optional[DecodeWorkspace] = None
        self._num_cus: Optional[int] = None
        # Out-of-range appends: the kernels skip a token whose cache position
        # or RoPE row is outside the tables and set this device flag; an eager
        # call reads it back asynchronously (pinned copy + event) and the next
        # eager call raises, as would mla.py:413's slice assignment.
        self._err: Optional[list] = None  # [device flag int32[1], pinned host copy, event or None]
        self._mask_ok = None  # (key, tensor) of the last mask verified as the prompt's causal mask
        # Split-KV plan of decode launches: "auto" balances the rows' splits
        # over the CUs on the device when positions come as a tensor (ragged
        # batches), "static" always cuts each row by its own length (the plan
        # an int start_pos gets: all rows alike), "balanced" always balances.
        self.split_plan = "auto"
        # A decode loop replayed from a HIP graph keeps its positions in a
        # device tensor and advances it after every step.  With this set, the
        # call itself adds T (its tokens per sequence) to a start_pos tensor
        # after its kernels have read it: a one-token step on the fused path
        # does it inside its last launch (wo's product), other calls with an
        # in-place add.  Meant for the last MLA a step runs.
        self.advance_positions = False
        self._advance_folded = False

    # ------------------------------------------------------------------ cache
    @property
    def fp8_cache(self) -> bool:
        return self.cache_dtype == "fp8_e4m3"

    def _param_like(self) -> torch.Tensor:
        return self.wkv_a.weight

    def set_inference_mode(self, mode: bool = True) -> None:
        """mla.py:184-225: allocate (True) or delete (False) the latent cache."""
        if mode == self.inference_mode:
            return
        self.inference_mode = mode
        if mode:
            # __init__ assigns plain None attributes; register_buffer refuses to
            # replace those (the reference's set_inference_mode raises KeyError
            # here, mla.py:180-182 vs :209), so drop them first.
            for name in ("kv_cache", "pe_cache", "kv_scale"):
                if name in self.__dict__ and self.__dict__[name] is None:
                    del self.__dict__[name]
            if self.attn_impl == "naive":
                raise NotImplementedError("attn_impl='naive' (full K/V cache) is not built")
            p = self._param_like()
            if getattr(self, "kv_cache", None) is None:
                shape = (self.max_batch_size, self.max_seq_len)
                if self.fp8_cache:
                    self.register_buffer(
                        "kv_cache",
                        torch.zeros(*shape, self.rank_pad, dtype=torch.uint8, device=p.device),
                        persistent=False,
                    )
                    self.register_buffer(
                        "kv_scale", torch.zeros(*shape, dtype=torch.float32, device=p.device), persistent=False
                    )
                else:
                    self.register_buffer(
                        "kv_cache",
                        torch.zeros(*shape, self.rank_pad, dtype=p.dtype, device=p.device),
                        persistent=False,
                    )
            if getattr(self, "pe_cache", None) is None:
                self.register_buffer(
                    "pe_cache",
                    torch.zeros(
                        self.max_batch_size, self.max_seq_len, self.qk_rope_head_dim, dtype=p.dtype, device=p.device
                    ),
                    persistent=False,
                )
        else:
            for name in ("k_cache", "v_cache", "kv_cache", "pe_cache", "kv_scale"):
                if hasattr(self, name):
                    delattr(self, name)

    def clear_cache(self) -> None:
        """mla.py:685-693, and leave inference mode so caches are reallocated."""
        for name in ("k_cache", "v_cache", "kv_cache", "pe_cache", "kv_scale"):
            if name in self._buffers:
                del self._buffers[name]
            setattr(self, name, None)
        self.inference_mode = False
        self._workspace = None

    def _apply(self, fn, recurse=True):
        # The e4m3 scale stays fp32 whatever dtype the module is cast to; it
        # only follows the module's device.
        scale = self._buffers.pop("kv_scale", None)
        try:
            out = super()._apply(fn, recurse)
        finally:
            if scale is not None:
                moved = fn(scale)
                self._buffers["kv_scale"] = scale.to(device=moved.device)
        return out

    # ------------------------------------------------------------ errors
    def _err_flag(self, device) -> Optional[torch.Tensor]:
        if self._err is None or self._err[0].device != device:
            if self._capturing():  # created by an eager call only (a captured zero-fill would rerun)
                return None
            flag = torch.zeros(1, dtype=torch.int32, device=device)
            self._err = [flag, torch.zeros(1, dtype=torch.int32, pin_memory=True), None]
        return self._err[0]

    @staticmethod
    def _capturing() -> bool:
        return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()

    def _raise_cache_error(self) -> None:
        flag, host, _ = self._err
        flag.zero_()
        host.zero_()
        self._err[2] = None
        raise RuntimeError(
            "an earlier call appended a token outside the latent cache or the RoPE table "
            "(start_pos + seqlen > max_seq_len, a negative start_pos, or a batch row past max_batch_size); "
            "those tokens were not written (mla.py:413 raises for the same input)")

    def _poll_cache_errors(self) -> None:
        """Raise for a flag an earlier eager call left set, if its read-back
        has landed (no synchronisation; skipped under graph capture)."""
        if self._err is None or self._capturing():
            return
        ev = self._err[2]
        if ev is not None and ev.query() and int(self._err[1][0]) != 0:
            self._raise_cache_error()

    def _read_back_cache_errors(self) -> None:
        if self._err is None or self._capturing():
            return
        flag, host, _ = self._err
        host.copy_(flag, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self._err[2] = ev

    def check_cache_errors(self) -> None:
        """Synchronising check: raise RuntimeError if any append since the
        last check skipped an out-of-range token (including appends replayed
        from a captured HIP graph), and clear the flag."""
        if self._err is None:
            return
        if int(self._err[0].item()) != 0:
            self._raise_cache_error()
        self._err[1].zero_()
        self._err[2] = None

    def latent_cache(self) -> LatentCache:
        """The module's cache buffers as a kernel-level ``LatentCache``."""
        if self.kv_cache is None or self.pe_cache is None:
            raise RuntimeError("no latent cache: call set_inference_mode(True) first")
        dt = self._param_like().dtype
        if self.pe_cache.dtype != dt or (not self.fp8_cache and self.kv_cache.dtype != dt):
            raise RuntimeError(
                f"cache dtype ({self.kv_cache.dtype}/{self.pe_cache.dtype}) does not match the "
                f"parameters ({dt}); convert the module before set_inference_mode(True)"
            )
        return LatentCache(self.kv_cache, self.pe_cache, self.kv_scale if self.fp8_cache else None,
                           self.kv_lora_rank)

    @property
    def rank_pad(self) -> int:
        """Latent channels stored per token: kv_lora_rank rounded up to 64."""
        return kernels.padded_rank(self.kv_lora_rank)

    def _padded(self, name: str, src: torch.Tensor, build) -> torch.Tensor:
        """A derived weight, rebuilt when ``src`` changes: ``build()`` pads it
        to R_pad; ``src`` itself is used when kv_lora_rank needs no padding."""
        if self.rank_pad == self.kv_lora_rank:
            return src.detach()
        return self._derived(name, src, build)

    def _derived(self, name: str, src: torch.Tensor, build) -> torch.Tensor:
        """``build()``, cached under ``name`` until ``src`` changes."""
        key = (src.data_ptr(), src._version, src.dtype, src.device)
        hit = self._padded_w.get(name)
        if hit is None or hit[0] != key:
            hit = (key, build().contiguous())
            self._padded_w[name] = hit
        return hit[1]

    def kv_norm_params(self) -> tuple[torch.Tensor, torch.Tensor]:
        """kv_norm's weight and bias zero-padded to R_pad (the kernels read
        R_pad entries; the padding takes no part in the LayerNorm)."""
        R = self.kv_lora_rank
        w = self._padded("kv_norm.weight", self.kv_norm.weight,
                         lambda: kernels.pad_rank(self.kv_norm.weight.detach(), R))
        b = self._padded("kv_norm.bias", self.kv_norm.bias,
                         lambda: kernels.pad_rank(self.kv_norm.bias.detach(), R))
        return w, b

    def _wkv_a_padded(self) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
        """wkv_a with its R latent rows followed by R_pad - R zero rows, so its
        output rows are [R_pad latent | P rope], the append kernels' layout."""
        R, rp, P = self.kv_lora_rank, self.rank_pad, self.qk_rope_head_dim

        def pad_rows(t):
            out = torch.zeros((rp + P,) + tuple(t.shape[1:]), dtype=t.dtype, device=t.device)
            out[:R] = t[:R]
            out[rp:] = t[R:]
            return out

        w = self._padded("wkv_a.weight", self.wkv_a.weight, lambda: pad_rows(self.wkv_a.weight.detach()))
        b = None
        if self.wkv_a.bias is not None:
            b = self._padded("wkv_a.bias", self.wkv_a.bias, lambda: pad_rows(self.wkv_a.bias.detach()))
        return w, b

    def _w_uv(self) -> torch.Tensor:
        """W_uv [H, Dv, R_pad] for mla_merge_project: a view of wkv_b.weight,
        or its zero-padded copy."""
        H, Dn, Dv, R = self.n_heads, self.qk_nope_head_dim, self.v_head_dim, self.kv_lora_rank
        view = lambda: self.wkv_b.weight.detach().view(H, Dn + Dv, R)[:, Dn:, :]
        if self.rank_pad == R:
            return view()
        return self._padded("w_uv", self.wkv_b.weight, lambda: kernels.pad_rank(view(), R))

    def _w_uv_fused(self) -> torch.Tensor:
        """_w_uv() over the fused step's heads (zero for the padding heads)."""
        H = self.n_heads
        Hp = self._fused_heads() or H
        if Hp == H:
            return self._w_uv()
        w_uv = self._w_uv()
        return self._derived("w_uv.fused", self.wkv_b.weight,
                             lambda: torch.cat([w_uv, w_uv.new_zeros((Hp - H,) + tuple(w_uv.shape[1:]))], 0))

    def _w_uk_t(self) -> torch.Tensor:
        """W_uk^T [H, R_pad, nope] for mla_head_product (its rows are the
        latent channels; zero beyond kv_lora_rank)."""
        w = self.wkv_b.weight
        key = (w.data_ptr(), w._version, w.dtype, w.device)
        hit = self._padded_w.get("w_uk_t")
        if hit is None or hit[0] != key:
            H, Dn, R = self.n_heads, self.qk_nope_head_dim, self.kv_lora_rank
            w_uk = kernels.pad_rank(w.detach().view(H, -1, R)[:, :Dn], R)  # [H, Dn, R_pad]
            hit = (key, w_uk.transpose(1, 2).contiguous())
            self._padded_w["w_uk_t"] = hit
        return hit[1]

    # ------------------------------------------------------------- weights
    def absorbed_weights(self) -> tuple[torch.Tensor, torch.Tensor]:
        """W_uk [H, nope, R_pad] and W_uv^T [H, R_pad, v] from wkv_b
        (mla.py:404-406, :427, :433), zero beyond kv_lora_rank."""
        w = self.wkv_b.weight
        key = (w.data_ptr(), w._version, w.dtype, w.device)
        if self._absorbed is None or self._absorbed[0] != key:
            R = self.kv_lora_rank
            wv = w.detach().view(self.n_heads, -1, R)
            w_uk = kernels.pad_rank(wv[:, : self.qk_nope_head_dim], R).contiguous()
            w_uv_t = kernels.pad_rank(wv[:, -self.v_head_dim:].transpose(1, 2), R, dim=1).contiguous()
            self._absorbed = (key, w_uk, w_uv_t)
        return self._absorbed[1], self._absorbed[2]

    def decode_weights(self) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
        """Stacked weight of the fused decode-step input product, rows
        [W_uk[h]^T . wq_nope[h] for every head (H*R_pad) | wq_pe (H*P) | wkv_a
        (R_pad+P)] over the model width, and its stacked bias (or None); the
        rows of the latent padding are zero.  One
        product x . W^T then yields q_abs = q_nope . W_uk (the absorbed query,
        re-associating mla.py:427), q_pe and the wkv_a rows (mla.py:281-288,
        :307).  The absorbed block is formed in fp32 and rounded once to the
        model dtype; rebuilt when any source weight changes."""
        ws = (self.wq.weight, self.wkv_a.weight, self.wkv_b.weight, self.wq.bias, self.wkv_a.bias)
        key = tuple(None if t is None else (t.data_ptr(), t._version, t.dtype, t.device) for t in ws)
        if self._decode_w is None or self._decode_w[0] != key:
            H, Dn, R, rp = self.n_heads, self.qk_nope_head_dim, self.kv_lora_rank, self.rank_pad
            Hp = self._fused_heads() or H  # heads past H: zero rows (padding to a launch's 16 heads)
            wq = self.wq.weight.detach().view(H, self.qk_head_dim, self.dim)
            w_uk = kernels.pad_rank(self.wkv_b.weight.detach().view(H, -1, R)[:, :Dn].float(), R)  # [H, Dn, R_pad]
            w_abs = torch.bmm(w_uk.transpose(1, 2).contiguous(), wq[:, :Dn].float().contiguous())
            w_pe = wq[:, Dn:].float()
            if Hp > H:
                w_abs = torch.cat([w_abs, w_abs.new_zeros((Hp - H,) + tuple(w_abs.shape[1:]))], 0)
                w_pe = torch.cat([w_pe, w_pe.new_zeros((Hp - H,) + tuple(w_pe.shape[1:]))], 0)
            wkv_a, bkv_a = self._wkv_a_padded()
            w_in = torch.cat(
                [w_abs.reshape(Hp * rp, self.dim), w_pe.reshape(-1, self.dim), wkv_a.float()], 0,
            ).to(self.wq.weight.dtype).contiguous()
            b_in = None
            if self.wq.bias is not None and self.wkv_a.bias is not None:
                bq = self.wq.bias.detach().view(H, self.qk_head_dim)
                b_abs = torch.bmm(bq[:, None, :Dn].float(), w_uk).reshape(H * rp)
                b_pe = bq[:, Dn:].float().reshape(-1)
                if Hp > H:
                    b_abs = torch.cat([b_abs, b_abs.new_zeros((Hp - H) * rp)])
                    b_pe = torch.cat([b_pe, b_pe.new_zeros((Hp - H) * (self.qk_head_dim - Dn))])
                b_in = torch.cat([b_abs, b_pe, bkv_a.float()]).to(self.wq.bias.dtype).contiguous()
            wp = None
            if w_in.is_cuda and kernels.packed_ok(1, w_in.shape[0], w_in.shape[1]):
                wp = kernels.pack_weight(w_in)
            self._decode_w = (key, w_in, b_in, wp)
        return self._decode_w[1], self._decode_w[2]

    def _wo_fused(self) -> torch.Tensor:
        """wo.weight over the fused step's heads: its own columns, followed by
        zero columns for the padding heads (whose read-out is zero)."""
        H, Dv = self.n_heads, self.v_head_dim
        Hp = self._fused_heads() or H
        if Hp == H:
            return self.wo.weight.detach()
        w = self.wo.weight.detach()
        return self._derived("wo.weight.fused", self.wo.weight,
                             lambda: torch.cat([w, w.new_zeros(w.shape[0], (Hp - H) * Dv)], 1))

    def _packed_wo(self) -> Optional["kernels.PackedWeight"]:
        """_wo_fused() in mla_linear_packed's layout (None when its shape is
        not covered); rebuilt when the weight changes."""
        w = self.wo.weight
        key = (w.data_ptr(), w._version, w.dtype, w.device, self._fused_heads())
        if self._wo_packed is None or self._wo_packed[0] != key:
            wp = None
            wf = self._wo_fused()
            if wf.is_cuda and wf.dtype == torch.bfloat16 and kernels.packed_ok(1, wf.shape[0], wf.shape[1]):
                wp = kernels.pack_weight(wf)
            self._wo_packed = (key, wp)
        return self._wo_packed[1]

    def _fused_projections(self, x: torch.Tensor):
        """q_abs [n, H, R_pad], q_pe [n, H, P] and kv [n, R_pad+P] from one
        product over decode_weights() (column views of one
        [n, H*(R_pad+P)+R_pad+P] buffer): mla_linear_packed with its packed
        copy while its grid fits the CUs in one round; past that (config 5's
        128 rows: 340 workgroups) the library GEMM (hipBLASLt through
        torch.nn.functional.linear) is faster, 9.4 against 15.1 us at 128 x 5440 x 1024; else
        mla_linear."""
        n, H, R, P = x.shape[0] * x.shape[1], self._fused_heads() or self.n_heads, self.rank_pad, self.qk_rope_head_dim
        xf = x.reshape(n, self.dim)
        if self.q_lora_rank > 0:
            # wq_a with wkv_a in one product, q_norm, then wq_b with W_uk absorbed
            (w1, b1, w1p), (w2, b2, w2p) = self._decode_weights_lora()
            y1 = self._product(xf, w1, b1, w1p)
            ql = self.q_lora_rank
            qn = torch.nn.functional.layer_norm(y1[:, :ql], (ql,), self.q_norm.weight, self.q_norm.bias,
                                                self.q_norm.eps)  # mla.py:102, :286
            y = self._product(qn, w2, b2, w2p)
            return y[:, : H * R].view(n, H, R), y[:, H * R:].view(n, H, P), y1[:, ql:]
        w_in, b_in = self.decode_weights()
        y = self._product(xf, w_in, b_in, self._decode_w[3])
        q_abs = y[:, : H * R].view(n, H, R)
        q_pe = y[:, H * R: H * (R + P)].view(n, H, P)
        return q_abs, q_pe, y[:, H * (R + P):]

    def _product(self, x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor],
                 wp: Optional["kernels.PackedWeight"]) -> torch.Tensor:
        """x . w^T (+ b) for the decode step: mla_linear_packed with the packed
        copy while its grid fits the CUs in one round; past that, or for a K
        the kernels do not take, the library GEMM; else mla_linear."""
        n, K = x.shape
        if wp is not None and kernels.packed_ok(n, wp.N, wp.K):
            if self._num_cus is None:
                self._num_cus = torch.cuda.get_device_properties(x.device).multi_processor_count
            if kernels.packed_blocks(n, wp.N, wp.K) <= self._num_cus:
                return kernels.linear_packed(x, wp, bias=b)
            return torch.nn.functional.linear(x, w, b)
        if K % 128 == 0 and x.stride(1) == 1:
            return kernels.linear(x, w, bias=b)
        return torch.nn.functional.linear(x, w, b)

    def _decode_weights_lora(self):
        """The q low-rank module's two stacked decode-step weights, each as
        (weight, bias or None, packed copy or None): [wq_a | wkv_a (R_pad +
        P rows)] over the model width, and [W_uk[h]^T . wq_b_nope[h] per head
        (padded to the fused step's heads) | wq_b_pe] over q_lora_rank (the
        absorbed block formed in fp32, rounded once)."""
        ws = (self.wq_a.weight, self.wq_b.weight, self.wkv_a.weight, self.wkv_b.weight, self.wq_a.bias,
              self.wq_b.bias, self.wkv_a.bias)
        key = tuple(None if t is None else (t.data_ptr(), t._version, t.dtype, t.device) for t in ws)
        if self._decode_w is None or self._decode_w[0] != key:
            H, Dn, R, rp, ql = self.n_heads, self.qk_nope_head_dim, self.kv_lora_rank, self.rank_pad, self.q_lora_rank
            Hp = self._fused_heads() or H
            dt = self.wq_a.weight.dtype
            wkv_a, bkv_a = self._wkv_a_padded()
            w1 = torch.cat([self.wq_a.weight.detach(), wkv_a], 0).to(dt).contiguous()
            b1 = None
            if self.wq_a.bias is not None:
                b1 = torch.cat([self.wq_a.bias.detach(), bkv_a]).to(dt).contiguous()
            wqb = self.wq_b.weight.detach().view(H, self.qk_head_dim, ql)
            w_uk = kernels.pad_rank(self.wkv_b.weight.detach().view(H, -1, R)[:, :Dn].float(), R)  # [H, Dn, R_pad]
            w_abs = torch.bmm(w_uk.transpose(1, 2).contiguous(), wqb[:, :Dn].float().contiguous())  # [H, R_pad, ql]
            w_pe = wqb[:, Dn:].float()
            if Hp > H:
                w_abs = torch.cat([w_abs, w_abs.new_zeros((Hp - H,) + tuple(w_abs.shape[1:]))], 0)
                w_pe = torch.cat([w_pe, w_pe.new_zeros((Hp - H,) + tuple(w_pe.shape[1:]))], 0)
            w2 = torch.cat([w_abs.reshape(Hp * rp, ql), w_pe.reshape(-1, ql)], 0).to(dt).contiguous()
            b2 = None
            if self.wq_b.bias is not None:
                bq = self.wq_b.bias.detach().view(H, self.qk_head_dim)
                b_abs = torch.bmm(bq[:, None, :Dn].float(), w_uk).reshape(H * rp)
                b_pe = bq[:, Dn:].float().reshape(-1)
                if Hp > H:
                    b_abs = torch.cat([b_abs, b_abs.new_zeros((Hp - H) * rp)])
                    b_pe = torch.cat([b_pe, b_pe.new_zeros((Hp - H) * (self.qk_head_dim - Dn))])
                b2 = torch.cat([b_abs, b_pe]).to(dt).contiguous()
            pk = lambda w: kernels.pack_weight(w) if (w.is_cuda and kernels.packed_ok(1, w.shape[0], w.shape[1])) else None
            self._decode_w = (key, (w1, b1, pk(w1)), (w2, b2, pk(w2)))
        return self._decode_w[1], self._decode_w[2]

    def _decode_heads(self) -> int:
        """Heads one decode launch takes for this module: all 32 of a bf16
        module at R_pad <= 256 (each wave serves both head groups from one
        stream of the cache), else 16."""
        if (self.n_heads == 32 and self.rank_pad <= 256
                and self.wkv_a.weight.dtype == torch.bfloat16):
            return 32
        return kernels.H

    def _fused_heads(self) -> Optional[int]:
        """Heads of the fused step's launches: the module's own 16 or 32 (as
        one decode launch takes them), 16 for fewer heads (zero-padded: the
        padding heads' query rows, read-out and wo columns are zero), else
        None."""
        if self.n_heads == self._decode_heads():
            return self.n_heads
        if self.n_heads < kernels.H:
            return kernels.H
        return None

    def _fused_step_ok(self, x: torch.Tensor, n: int) -> bool:
        """The decode-step kernels cover bf16 modules with up to 16 heads (or
        32, in one launch), kv_lora_rank up to 512, at most 128 query rows and
        128-aligned model widths; a q low-rank module runs its query through
        two products with q_norm between them."""
        wq = self.wq if self.q_lora_rank == 0 else self.wq_a
        q_bias = (wq.bias is not None) if self.q_lora_rank == 0 else (
            (self.wq_a.bias is not None) and (self.wq_b.bias is not None))
        return (
            self._fused_heads() is not None
            and self.rank_pad <= kernels.MFMA_MAX_RANK
            and x.dtype == torch.bfloat16
            and wq.weight.dtype == torch.bfloat16
            and 0 < n <= kernels.LINEAR_MAX_ROWS
            and self.dim % 128 == 0
            and (self.n_heads * self.v_head_dim) % 128 == 0
            and q_bias == (self.wkv_a.bias is not None)
            and self.v_head_dim == 128
        )

    def _check_geometry(self) -> None:
        if (self.n_heads < 1 or self.qk_rope_head_dim != kernels.P
                or not 1 <= self.kv_lora_rank <= kernels.MAX_RANK):
            raise NotImplementedError(
                f"kernels are built for qk_rope_head_dim={kernels.P} and kv_lora_rank 1..{kernels.MAX_RANK} "
                f"(any n_heads); got n_heads={self.n_heads}, kv_lora_rank={self.kv_lora_rank}, "
                f"qk_rope_head_dim={self.qk_rope_head_dim}"
            )

    def _split_plan(self, n_rows: int, max_len: int, device, blocks_per_cu: int = 1) -> tuple[int, int]:
        if self._num_cus is None:
            self._num_cus = torch.cuda.get_device_properties(device).multi_processor_count
        return kernels.plan_splits(n_rows, max_len, num_cus=self._num_cus, blocks_per_cu=blocks_per_cu)

    def _decode_plan(self, n_rows: int, max_len: int, device, per_row_positions: bool,
                     dtype: Optional[torch.dtype] = None) -> tuple[int, int, int]:
        """(n_splits, min_chunk, balance) of a decode launch, sized for as many
        workgroups as the CUs hold at once (one per CU for a bf16 cache, three
        for an e4m3 cache at ranks up to 256).  With per-sequence positions (a
        start_pos tensor: lengths unknown to the host, ragged in general) the
        launch balances the rows' splits over those slots from the lengths on
        the device, so the plan follows them in a replayed graph;
        ``split_plan`` overrides the choice."""
        if self.split_plan not in ("auto", "static", "balanced"):
            raise ValueError(f"split_plan must be 'auto', 'static' or 'balanced', got {self.split_plan!r}")
        dt = dtype if dtype is not None else self.wkv_a.weight.dtype
        fused = dt == torch.bfloat16 and self.rank_pad <= kernels.MFMA_MAX_RANK
        bpc = kernels.decode_blocks_per_cu(dt, self.fp8_cache, self.kv_lora_rank, fused, device)
        n_splits, min_chunk = self._split_plan(n_rows, max_len, device, bpc)
        if self.split_plan == "balanced" or (self.split_plan == "auto" and per_row_positions):
            bal, cap = kernels.balanced_splits(n_rows, self._num_cus, bpc)
            if bal:
                return cap, min_chunk, bal
        return n_splits, min_chunk, 0

    def _workspace_for(self, n_rows: int, n_splits: int, device, heads: int = kernels.H) -> Optional[DecodeWorkspace]:
        if n_splits <= 1:
            return None
        ws = self._workspace
        if ws is None or not ws.fits(n_rows, n_splits, self.kv_lora_rank, heads) or ws.o_part.device != device:
            ws = DecodeWorkspace.allocate(n_rows, n_splits, device, rank=self.kv_lora_rank, heads=heads)
            self._workspace = ws
        return ws

    # ------------------------------------------------------------- forward
    def forward(
        self,
        x: torch.Tensor,
        start_pos: Union[int, torch.Tensor],
        freqs_cis: Optional[torch.Tensor] = None,
        mask: Optional[torch.Tensor] = None,
        position_ids: Optional[torch.Tensor] = None,
        cu_seqlens: Optional[torch.Tensor] = None,
        max_seqlen: Optional[int] = None,
    ) -> torch.Tensor:
        """mla.py:232-495 (absorb branch).  ``freqs_cis`` is ignored exactly as
        in the reference's RoPE call (positional_encoding.py:30-34)."""
        if self.training and self.inference_mode:  # mla.py:274-275
            self.set_inference_mode(False)
        if position_ids is not None or cu_seqlens is not None:
            raise NotImplementedError("position_ids / cu_seqlens backends are not part of this path")
        if mask is not None and not self._is_causal_prompt_mask(mask, x.size(1), start_pos):
            raise NotImplementedError(
                "only the additive causal mask of a prompt at start_pos 0 (swa_mla_model.py:384-387) is "
                "supported; other masks are not part of this path")
        if self.attn_impl != "absorb":
            raise NotImplementedError(f"attn_impl={self.attn_impl!r} is not built")
        if torch.is_grad_enabled() and x.requires_grad:
            raise NotImplementedError("the training / autograd path is not part of this build")
        if x.device.type != "cuda":
            raise RuntimeError("swamla_amd.MLA runs on the GPU only (no CPU fallback)")
        if self.advance_positions and not isinstance(start_pos, torch.Tensor):
            raise ValueError("advance_positions needs start_pos as a tensor (an int cannot be advanced in place)")
        self._check_geometry()
        self._poll_cache_errors()
        self._advance_folded = False
        with torch.no_grad():
            out = self._forward_kernels(x, start_pos)
            if self.advance_positions and not self._advance_folded:
                start_pos.add_(x.size(1))
        self._read_back_cache_errors()
        return out

    def _advance_target(self, start_pos, sp: torch.Tensor, T: int) -> Optional[torch.Tensor]:
        """The positions tensor a one-token step's last launch may advance
        itself: start_pos's own storage as the kernels read it (int32,
        contiguous, at most 512 entries), else None (forward adds in place)."""
        if not (self.advance_positions and T == 1 and isinstance(start_pos, torch.Tensor)):
            return None
        if (start_pos.dtype != torch.int32 or not start_pos.is_contiguous() or sp.data_ptr() != start_pos.data_ptr()
                or not 1 <= sp.numel() <= 512):
            return None
        return sp

    def _is_causal_prompt_mask(self, mask: torch.Tensor, T: int, start_pos) -> bool:
        """True for the mask SWAMLAModel passes with a prompt
        (swa_mla_model.py:207-211, :384-387: triu(full(-inf), 1)[:T, :T],
        additive) when the call starts at position 0, where the reference's
        SDPA with that mask (mla.py:473-485) equals the causal attention the
        kernels run.  Verified once per mask tensor (a device comparison,
        so not under graph capture)."""
        if isinstance(start_pos, torch.Tensor) or int(start_pos) != 0:
            return False
        if mask.dim() != 2 or tuple(mask.shape) != (T, T) or not mask.is_floating_point():
            return False
        # the verified tensor is kept alive with its key, so an equal pointer is
        # the same storage and an equal version means it was not written since
        key = (mask.data_ptr(), mask.device, mask.dtype, tuple(mask.stride()), mask._version, T)
        if self._mask_ok is not None and self._mask_ok[0] == key:
            return True
        if self._capturing():
            return False
        want = torch.full((T, T), float("-inf"), dtype=mask.dtype, device=mask.device).triu(1)
        if not torch.equal(mask, want):
            return False
        self._mask_ok = (key, mask)
        return True

    def prefill_cache(self, x: torch.Tensor, start_pos: Union[int, torch.Tensor] = 0) -> None:
        """Append path only (wkv_a GEMM + fused append kernel), no attention:
        writes the latent / k_pe rows of the T tokens of ``x`` into the cache,
        exactly as ``forward`` would (mla.py:307-323, :409-414)."""
        if not self.inference_mode:
            raise RuntimeError("prefill_cache needs set_inference_mode(True)")
        if x.device.type != "cuda":
            raise RuntimeError("swamla_amd.MLA runs on the GPU only (no CPU fallback)")
        self._check_geometry()
        B, T, _ = x.size()
        self._poll_cache_errors()
        cache = self.latent_cache()
        sp = self._start_positions(B, T, start_pos, cache, x.device)
        with torch.no_grad():
            _, kv = self.input_projections(x, need_q=False)
            cos, sin = self.rope.half_tables()
            ln_w, ln_b = self.kv_norm_params()
            kernels.append(kv, cache, ln_w, ln_b, self.kv_norm.eps, cos, sin,
                           start_pos=sp, tokens_per_seq=T, rope_abs=self.rope_positions == "absolute",
                           err_flag=self._err_flag(x.device))
        self._read_back_cache_errors()

    def input_projections(self, x: torch.Tensor, need_q: bool = True) -> tuple[Optional[torch.Tensor], torch.Tensor]:
        """(q [B*T, H, 192] or None, kv [B*T, R_pad + P]): the wkv_a rows
        that forward feeds the append kernel (mla.py:281-288, :307-308), with
        zero latent padding up to R_pad.
        Decode-sized bf16 inputs take kv from the fused input product (and
        return no q: forward uses the absorbed query directly); other inputs
        use the ATen projections (q is skipped when not needed)."""
        B, T, _ = x.size()
        n, H = B * T, self.n_heads
        with torch.no_grad():
            if self._fused_step_ok(x, n):
                _, _, kv = self._fused_projections(x)
                return None, kv
            if self.rank_pad == self.kv_lora_rank:
                kv = self.wkv_a(x).view(n, -1)
            else:
                w, b = self._wkv_a_padded()
                kv = torch.nn.functional.linear(x, w, b).view(n, -1)
            if not need_q:
                return None, kv
            if self.q_lora_rank == 0:
                q = self.wq(x)
            else:
                q = self.wq_b(self.q_norm(self.wq_a(x)))
            return q.view(n, H, self.qk_head_dim), kv

    def _start_positions(self, B: int, T: int, start_pos, cache: LatentCache, device) -> torch.Tensor:
        """int32 [B] device tensor of per-sequence start positions (checked
        against the cache when given as an int, as mla.py:413 would raise)."""
        if B > cache.ckv.shape[0]:
            raise ValueError(f"batch {B} exceeds max_batch_size {cache.ckv.shape[0]}")
        if isinstance(start_pos, torch.Tensor):
            if start_pos.numel() != B:
                raise ValueError(f"start_pos tensor has {start_pos.numel()} entries for batch {B}")
            if start_pos.device.type == "cpu":  # values known on the host: check them now
                lo_, hi_ = int(start_pos.min()), int(start_pos.max())
                if lo_ < 0 or hi_ + T > cache.ckv.shape[1]:
                    raise ValueError(f"start_pos in [{lo_}, {hi_}] + seqlen {T} is outside max_seq_len "
                                     f"{cache.ckv.shape[1]}")
            # device values are checked by the kernels (the module's error flag)
            sp = start_pos.to(device=device, dtype=torch.int32).reshape(-1)
            return sp if sp.is_contiguous() else sp.contiguous()
        start_pos = int(start_pos)
        if start_pos < 0 or start_pos + T > cache.ckv.shape[1]:
            raise ValueError(f"start_pos {start_pos} + seqlen {T} exceeds max_seq_len {cache.ckv.shape[1]}")
        return torch.full((B,), start_pos, dtype=torch.int32, device=device)

    def _forward_kernels(self, x: torch.Tensor, start_pos) -> torch.Tensor:
        B, T, _ = x.size()
        dev = x.device
        H, R, Dn, Dv = self.n_heads, self.kv_lora_rank, self.qk_nope_head_dim, self.v_head_dim
        n = B * T
        rope_abs = self.rope_positions == "absolute"

        if self.inference_mode:
            cache = self.latent_cache()
            sp = self._start_positions(B, T, start_pos, cache, dev)
            max_len = (int(start_pos) + T) if not isinstance(start_pos, torch.Tensor) else cache.ckv.shape[1]
        else:
            # No cache (mla.py:419-423): attend over this call's tokens only.
            if T > self.rope.cos_cached.shape[2]:
                # The table grows to T positions in fp32 (positional_encoding.py:44-46, :64-86). For an
                # fp32 module nothing else changes. For bf16 the reference's rotation then yields fp32
                # q_pe / k_pe, and its SDPA receives fp32 queries and keys with bf16 values and raises
                # (mla.py:555-601); this path raises before changing the table.
                if x.dtype != torch.float32 or self.rope.cos_cached.dtype != torch.float32:
                    raise ValueError(
                        f"seqlen {T} exceeds the RoPE table ({self.rope.cos_cached.shape[2]} positions): the "
                        f"table grows in fp32, which only an fp32 module can use (the reference's attention "
                        f"rejects the mixed dtypes that growth makes in a {x.dtype} module)")
                self.rope.extend(T)
            cache = LatentCache.allocate(B, T, x.dtype, dev, fp8=self.fp8_cache, rank=R)
            sp = torch.zeros(B, dtype=torch.int32, device=dev)
            max_len = T

        fused = self._fused_step_ok(x, n)
        if fused:
            q_abs, q_pe, kv = self._fused_projections(x)
        else:
            q, kv = self.input_projections(x)

        cos, sin = self.rope.half_tables()
        # A one-token step appends inside the attention launch; longer chunks
        # append first (their rows attend to each other's new tokens).
        fold_append = fused and T == 1
        ln_w, ln_b = self.kv_norm_params()
        err = self._err_flag(dev)
        if not fold_append:
            kernels.append(kv, cache, ln_w, ln_b, self.kv_norm.eps, cos, sin,
                           start_pos=sp, tokens_per_seq=T, rope_abs=rope_abs, err_flag=err)

        n_splits, min_chunk, balance = self._decode_plan(
            n, max_len, dev, isinstance(start_pos, torch.Tensor) and self.inference_mode, dtype=x.dtype)
        # A chunk of many tokens per sequence: four queries share each cache
        # tile (no split-KV) instead of one row per workgroup.
        prefill = x.dtype == torch.bfloat16 and kernels.use_prefill(B, T, self._num_cus, rank=R)
        if prefill:
            n_splits, balance = 1, 0
        if fused:
            Hp = self._fused_heads()  # the launches' heads: H, or 16 with zero padding heads
            o_lat = torch.empty(n, Hp, self.rank_pad, dtype=x.dtype, device=dev)
            ws = self._workspace_for(n, n_splits, dev, heads=Hp)
            if prefill:
                kernels.prefill_attention(q_abs, q_pe, cos, sin, cache, self.softmax_scale, start_pos=sp,
                                          rows_per_seq=T, rope_abs=rope_abs, out=o_lat)
            else:
                fa = None
                if fold_append:
                    fa = kernels.FusedAppend(kv, ln_w, ln_b, self.kv_norm.eps, err_flag=err)
                kernels.decode_attention(
                    q_abs, q_pe, cos, sin, cache, self.softmax_scale,
                    start_pos=sp, rows_per_seq=T, rope_abs=rope_abs, n_splits=n_splits, min_chunk=min_chunk,
                    out=o_lat, workspace=ws, merge=False, append=fa, balance=balance,
                )
            # o[r, h*Dv + d] = W_uv[h][d] . merged o_lat[r, h]: split merge and
            # read-out in one launch, written straight in wo's input layout
            w_uv = self._w_uv_fused()
            o = torch.empty(n, Hp * Dv, dtype=x.dtype, device=dev)
            kernels.merge_project(o_lat, w_uv, o.view(n, Hp, Dv), cache, n_splits=n_splits, min_chunk=min_chunk,
                                  workspace=ws, start_pos=sp, rows_per_seq=T, balanced=balance > 0)
            wo_b = None if self.wo.bias is None else self.wo.bias.detach()
            wo_p = self._packed_wo()
            if wo_p is not None and kernels.packed_ok(n, wo_p.N, wo_p.K):
                adv = self._advance_target(start_pos, sp, T)
                out = kernels.linear_packed(o, wo_p, bias=wo_b, advance=adv).view(B, T, self.dim)
                self._advance_folded = adv is not None
            else:
                out = kernels.linear(o, self._wo_fused(), bias=wo_b).view(B, T, self.dim)
            return self.resid_dropout(out)  # mla.py:490-495

        # Other calls: the absorbed products, then attention.  The attention
        # kernels take 16 heads per launch (the decode kernel also 32), so H
        # heads run as ceil(H / HK) launches over query rows padded with zero
        # heads (whose outputs are dropped).
        rp = self.rank_pad
        HK = self._decode_heads() if (not prefill and x.dtype == torch.bfloat16) else kernels.H
        Hp = -(-H // HK) * HK
        # prompt-sized bf16 calls: per-head MFMA products that read q and o_lat
        # in place and write q_abs in the attention kernels' layout and o in
        # wo's (re-associating mla.py:427, :433); fp32 modules use ATen's
        # batched products
        use_hp = (x.dtype == torch.bfloat16 and kernels.head_product_ok(Dn, rp)
                  and kernels.head_product_ok(rp, Dv))
        if Hp == H:
            q_abs = torch.empty(n, H, rp, dtype=x.dtype, device=dev)
            q_pe = q[:, :, Dn:]
        else:
            q_abs = torch.zeros(n, Hp, rp, dtype=x.dtype, device=dev)
            q_pe = torch.zeros(n, Hp, self.qk_rope_head_dim, dtype=x.dtype, device=dev)
            q_pe[:, :H] = q[:, :, Dn:]
        if use_hp:
            kernels.head_product(q[:, :, :Dn], self._w_uk_t(), out=q_abs[:, :H])  # [n, H, R_pad]
        else:
            w_uk, w_uv_t = self.absorbed_weights()
            q_nope = q[:, :, :Dn].transpose(0, 1).contiguous()  # [H, n, Dn]
            q_abs[:, :H] = torch.bmm(q_nope, w_uk).transpose(0, 1)  # [n, H, R_pad]
        o_lat = torch.empty(n, Hp, rp, dtype=x.dtype, device=dev)
        ws = None if prefill else self._workspace_for(n, n_splits, dev, heads=HK)
        for h0 in range(0, Hp, HK):
            hs = slice(h0, h0 + HK)
            if prefill:
                kernels.prefill_attention(q_abs[:, hs], q_pe[:, hs], cos, sin, cache, self.softmax_scale,
                                          start_pos=sp, rows_per_seq=T, rope_abs=rope_abs, out=o_lat[:, hs])
            else:
                kernels.decode_attention(
                    q_abs[:, hs], q_pe[:, hs], cos, sin, cache, self.softmax_scale,
                    start_pos=sp, rows_per_seq=T, rope_abs=rope_abs, n_splits=n_splits, min_chunk=min_chunk,
                    out=o_lat[:, hs], workspace=ws, balance=balance,
                )
        if use_hp:
            o = torch.empty(n, H * Dv, dtype=x.dtype, device=dev)
            kernels.head_product(o_lat[:, :H], self._w_uv(), out=o.view(n, H, Dv))
        else:
            o = torch.bmm(o_lat[:, :H].transpose(0, 1), w_uv_t).transpose(0, 1).reshape(n, H * Dv)  # [n, H*Dv]
        return self.resid_dropout(self.wo(o.view(B, T, H * Dv)))  # mla.py:490-495
