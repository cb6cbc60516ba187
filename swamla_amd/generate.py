"""Model-level incremental decoding over the drop-in MLA's latent caches.

The reference generates by re-running the whole context through the model
for every new token (SWAMLAModel.generate, models/swa_mla_model.py:507-552;
InferenceEngine.generate, inference.py:97-102): its forward passes start_pos
0 to every block (swa_mla_model.py:394-406).  ``IncrementalDecoder`` runs the
same model once over the prompt and then one token per step, threading each
MLA block's start position so the blocks attend over their latent caches.

Scope: models whose blocks are all MLA blocks holding ``swamla_amd.MLA``
(the reference's SWAMLAModel with ``local_layers_per_cycle = 0``).  A
GatedDeltaNet block would need its recurrent state carried between calls and
an Engram block its n-gram token history; both raise ``NotImplementedError``.

With ``graph=True`` the one-token steps after the first are replayed from a
HIP graph captured at the first step: the start position lives on the device
and the graph advances it, so a step costs one graph launch instead of the
host issuing every kernel (the positions are then a device tensor, which
gives the MLA's split plan the cache length instead of the exact one: the
same results up to summation order).

The model is used through the attributes SWAMLAModel has
(``transformer.wte / drop / h / ln_f``, ``lm_head``, ``config.block_size``)
and each block through its call ``block(x, start_pos, freqs_cis, mask)``
(models/mla_block.py:81).

Side effects on the model's MLA modules, undone by ``close()`` (or by leaving
a ``with IncrementalDecoder(model) as dec:`` block): they are switched to
absolute RoPE positions — a new token at position p must be rotated by p,
which is what the reference's full-context recompute does (its chunk-local
convention rotates a one-token call by 0) — and, for graph replays, to the
per-row split plan; while the graph is captured the last one advances the
device positions (``MLA.advance_positions``).  Their caches stay allocated (``MLA.clear_cache`` frees
them).

Positions are checked on the host against the smaller of ``block_size`` and
every MLA's cache length before each step, eager or replayed; after
``generate`` the modules' device-side append flags are read back as well.
"""
from __future__ import annotations

from typing import Optional

import torch

from .mla import MLA

__all__ = ["IncrementalDecoder"]


class IncrementalDecoder:
    def __init__(self, model, graph: bool = False):
        self.model = model
        self.graph = graph
        self._g = None  # (graph, token buffer [B, 1], device positions [B], logits buffer)
        self.blocks = list(model.transformer.h)
        self.mlas = []
        for i, blk in enumerate(self.blocks):
            attn = getattr(blk, "attn", None)
            if not isinstance(attn, MLA):
                raise NotImplementedError(
                    f"block {i} ({type(blk).__name__}) holds no swamla_amd.MLA: recurrent (DeltaNet) blocks "
                    "are not part of this path")
            if getattr(blk, "has_engram", False):
                raise NotImplementedError(f"block {i} has an Engram module, whose n-gram lookup needs the token "
                                          "history; not part of this path")
            self.mlas.append(attn)
        if not self.mlas:
            raise ValueError("the model has no blocks: nothing to decode incrementally")
        self.block_size = int(model.config.block_size)
        self.limit = self.block_size  # positions available: block_size and every cache length
        self.pos = 0
        # the attributes prefill() / the graph capture change, restored by close()
        self._saved = [(m, m.rope_positions, m.split_plan, m.advance_positions) for m in self.mlas]

    def close(self) -> None:
        """Restore each MLA's RoPE convention, split plan and position advance as they were
        before this decoder touched them, and drop the captured graph."""
        for m, rope_positions, split_plan, advance in self._saved:
            m.rope_positions = rope_positions
            m.split_plan = split_plan
            m.advance_positions = advance
        self._g = None

    def __enter__(self) -> "IncrementalDecoder":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def _check_room(self, t: int) -> None:
        if self.pos + t > self.limit:
            what = "block_size" if self.limit == self.block_size else "the smallest MLA cache length"
            raise ValueError(f"position {self.pos + t} exceeds {what} ({self.limit})")

    def _run(self, idx: torch.Tensor, start_pos) -> torch.Tensor:
        """Logits of the last position after running ``idx`` [B, T] from
        ``start_pos`` (an int, or an int32 device tensor [B] of positions;
        swa_mla_model.py:365-406 with start_pos threaded)."""
        t = idx.shape[1]
        self._check_room(t)
        tr = self.model.transformer
        x = tr.drop(tr.wte(idx))
        # the prompt's additive causal mask, as the model builds it (:384-387);
        # a one-token step attends to everything cached (mask None)
        mask = None
        if t > 1:
            mask = torch.triu(torch.full((t, t), float("-inf"), device=idx.device), diagonal=1)
        for blk in self.blocks:
            x = blk(x, start_pos, None, mask)
        x = tr.ln_f(x[:, -1:, :])
        return self.model.lm_head(x)[:, -1, :]

    @torch.no_grad()
    def prefill(self, idx: torch.Tensor) -> torch.Tensor:
        """Start a new sequence batch: caches (re)allocated, the prompt
        [B, T] appended at positions 0 .. T-1; returns the last logits."""
        for m in self.mlas:
            m.rope_positions = "absolute"
            if m.inference_mode and m.kv_cache is not None and m.kv_cache.shape[0] < idx.shape[0]:
                m.clear_cache()
            m.set_inference_mode(True)
        self.limit = min([self.block_size] + [int(m.kv_cache.shape[1]) for m in self.mlas])
        self.pos = 0
        self._g = None
        logits = self._run(idx, 0)
        self.pos = idx.shape[1]
        return logits

    @torch.no_grad()
    def step(self, idx_next: torch.Tensor) -> torch.Tensor:
        """Append one token per sequence ([B, 1]) and return its logits."""
        if idx_next.dim() != 2 or idx_next.shape[1] != 1:
            raise ValueError("step takes one token per sequence: [B, 1]")
        if not self.graph:
            logits = self._run(idx_next, self.pos)
            self.pos += 1
            return logits
        if self._g is not None:
            graph, tok, sp, out = self._g
            self._check_room(1)  # the replay's positions come from the device
            tok.copy_(idx_next)
            graph.replay()
            self.pos += 1
            return out.clone()
        # First step: run it eagerly with device positions on a side stream
        # (allocating the layers' workspaces), then capture the step for the
        # next ones; the captured step advances the positions itself.
        dev = idx_next.device
        tok = idx_next.clone()
        sp = torch.full((idx_next.shape[0],), self.pos, dtype=torch.int32, device=dev)
        for m in self.mlas:
            m.split_plan = "static"  # a uniform batch: each row cut by its own length
            m.advance_positions = False
        # the last MLA of the step advances the positions (inside its last
        # launch on the fused one-token path)
        self.mlas[-1].advance_positions = True
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            logits = self._run(tok, sp)
        torch.cuda.current_stream(dev).wait_stream(side)
        self.pos += 1
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = self._run(tok, sp)
        self.mlas[-1].advance_positions = False
        self._g = (graph, tok, sp, out)
        return logits

    @torch.no_grad()
    def generate(self, idx: torch.Tensor, max_new_tokens: int, temperature: float = 1.0,
                 top_k: Optional[int] = None, generator: Optional[torch.Generator] = None) -> torch.Tensor:
        """SWAMLAModel.generate's sampling (swa_mla_model.py:537-552) over
        incremental steps: returns idx with max_new_tokens tokens appended.
        Unlike the reference it does not slide the context past block_size
        (the caches hold the whole sequence); that raises ValueError."""
        logits = self.prefill(idx)
        out = idx
        for i in range(max_new_tokens):
            logits = logits / max(temperature, 1e-6)
            if top_k is not None:
                values, _ = torch.topk(logits, min(top_k, logits.size(-1)))
                logits[logits < values[:, [-1]]] = -float("inf")
            probs = torch.softmax(logits.float(), dim=-1)
            idx_next = torch.multinomial(probs, num_samples=1, generator=generator)
            out = torch.cat((out, idx_next), dim=1)
            if i + 1 < max_new_tokens:
                logits = self.step(idx_next)
        for m in self.mlas:
            m.check_cache_errors()  # appends skipped on the device (e.g. in graph replays) raise here
        return out
