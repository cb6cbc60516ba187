"""RoPE tables for the latent-cache path.

Reference: models/positional_encoding.py:9-28 (table), :30-62 (interleaved
rotation), :64-86 (growth), :88-91 (forward).  The table is built on the CPU in fp32 with the
same torch ops as the reference so every entry is bitwise identical, kept as
the same non-persistent buffers (``cos_cached`` / ``sin_cached``,
[1, 1, max_seq_len, dim]) so ``module.to(dtype)`` rounds it exactly as it
rounds the reference's.  The kernels read the first dim/2 columns as
[max_seq_len, dim/2] tables (the reference uses ``cos[..., :D//2]`` only).
The rotation itself runs inside the HIP kernels.
"""
from __future__ import annotations

import torch
import torch.nn as nn


def rope_tables(dim: int, max_seq_len: int, base: int = 10000) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos / sin tables [1, 1, max_seq_len, dim] (positional_encoding.py:21-28)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))
    t = torch.arange(max_seq_len).type_as(inv_freq)
    freqs = torch.einsum("i,j->ij", t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().view(1, 1, max_seq_len, dim), emb.sin().view(1, 1, max_seq_len, dim)


class RoPE(nn.Module):
    """Holds the reference's RoPE buffers; rotation happens in the kernels."""

    def __init__(self, dim: int, max_seq_len: int = 2048, base: int = 10000):
        super().__init__()
        self.dim = dim
        self.max_seq_len = max_seq_len
        self.base = base
        cos, sin = rope_tables(dim, max_seq_len, base)
        self.register_buffer("cos_cached", cos, persistent=False)
        self.register_buffer("sin_cached", sin, persistent=False)
        self._half = None  # (key, cos_half, sin_half)
        self._retired = []

    def extend(self, new_max_len: int) -> None:
        """Table growth (positional_encoding.py:44-46, :64-86): the table is
        rebuilt for new_max_len positions in fp32 on the buffers' device with
        the same torch ops, and replaces the buffers, whose dtype becomes fp32
        whatever the module's dtype was."""
        if new_max_len <= self.max_seq_len:
            return
        self.max_seq_len = new_max_len
        if self._half is not None:
            # graphs captured earlier may hold these tables' addresses
            self._retired.append(self._half)
            self._half = None
        dev = self.cos_cached.device
        inv_freq = (1.0 / (self.base ** (torch.arange(0, self.dim, 2).float() / self.dim))).to(dev)
        t = torch.arange(new_max_len, device=dev).type_as(inv_freq)
        freqs = torch.einsum("i,j->ij", t, inv_freq)
        emb = torch.cat((freqs, freqs), dim=-1)
        self.register_buffer("cos_cached", emb.cos().view(1, 1, new_max_len, self.dim), persistent=False)
        self.register_buffer("sin_cached", emb.sin().view(1, 1, new_max_len, self.dim), persistent=False)

    def half_tables(self) -> tuple[torch.Tensor, torch.Tensor]:
        """Contiguous [max_seq_len, dim/2] cos / sin in the buffers' dtype/device."""
        c, s = self.cos_cached, self.sin_cached
        key = (c.data_ptr(), s.data_ptr(), c.dtype, c.device)
        if self._half is None or self._half[0] != key:
            half = self.dim // 2
            self._half = (
                key,
                c[0, 0, :, :half].contiguous(),
                s[0, 0, :, :half].contiguous(),
            )
        return self._half[1], self._half[2]
