"""A small SWAMLAModel-shaped model for the incremental-decoding tests: the
attributes IncrementalDecoder uses (transformer.wte / drop / h / ln_f,
lm_head, config.block_size) and MLA blocks with the reference MLABlock's
residual structure (models/mla_block.py:153-158: x + attn(attn_norm(x)),
then x + ffn(ffn_norm(x))), RMSNorm as models/normalization.py:17-37 and a
SwiGLU MLP as models/mlp.py:19-49.  The attention module is passed in: the
drop-in swamla_amd.MLA or the oracle's RefMLA."""
from types import SimpleNamespace

import torch
import torch.nn as nn
import torch.nn.functional as F


class RMSNorm(nn.Module):
    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        if x.dtype in (torch.bfloat16, torch.float16):
            return self.weight * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps))
        return (self.weight * (x.float() * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + self.eps))).to(x.dtype)


class MLP(nn.Module):
    def __init__(self, dim):
        super().__init__()
        self.gate_up_proj = nn.Linear(dim, 8 * dim, bias=False)
        self.down_proj = nn.Linear(4 * dim, dim, bias=False)

    def forward(self, x):
        gate, up = self.gate_up_proj(x).chunk(2, dim=-1)
        return self.down_proj(F.silu(gate) * up)


class Block(nn.Module):
    def __init__(self, dim, attn):
        super().__init__()
        self.attn_norm = RMSNorm(dim)
        self.attn = attn
        self.ffn_norm = RMSNorm(dim)
        self.ffn = MLP(dim)

    def forward(self, x, start_pos=0, freqs_cis=None, mask=None):
        x = x + self.attn(self.attn_norm(x), start_pos, freqs_cis, mask)
        return x + self.ffn(self.ffn_norm(x))


class TinyModel(nn.Module):
    def __init__(self, vocab, dim, block_size, attns):
        super().__init__()
        self.config = SimpleNamespace(block_size=block_size)
        self.transformer = nn.ModuleDict(dict(
            wte=nn.Embedding(vocab, dim), drop=nn.Dropout(0.0),
            h=nn.ModuleList([Block(dim, a) for a in attns]), ln_f=RMSNorm(dim)))
        self.lm_head = nn.Linear(dim, vocab, bias=False)
        self.lm_head.weight = self.transformer.wte.weight

    def full_logits(self, idx):
        """The reference's per-token forward: the whole context from
        position 0 with the causal mask (swa_mla_model.py:365-406), logits of
        the last position."""
        t = idx.shape[1]
        x = self.transformer.drop(self.transformer.wte(idx))
        mask = torch.triu(torch.full((t, t), float("-inf"), device=idx.device), diagonal=1) if t > 1 else None
        for blk in self.transformer.h:
            x = blk(x, 0, None, mask)
        return self.lm_head(self.transformer.ln_f(x))[:, -1, :]
