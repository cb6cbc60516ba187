"""CPU oracle for the MLA latent-KV-cache path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker / the timed CPU
baseline.  The product path (``swamla_amd``) never imports it and has no CPU
fallback.

Contents
  mla_ref      op-for-op torch restatement of the reference ``MLA`` absorb
               branch and ``RoPE`` (models/mla.py, models/positional_encoding.py);
               pinned bit-exactly to the real reference by tests/golden fixtures.
  latent_ops   numpy / fp64 statements of what each kernel must produce:
               torch's CPU LayerNorm op for op (aten_layernorm.c), bf16 /
               e4m3 rounding, per-op-rounded RoPE, absorbed attention in fp64,
               split plan and log-sum-exp merge.  Each function's header says
               how it is pinned.
"""
