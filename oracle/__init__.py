"""CPU oracle for the block-sparse attention hot path -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s CPU-baseline leg may import this package, and only as
the checker (never as the thing measured or shipped). The product path (`self_trainable_or_free_attn_amd`) never
imports it and fails loudly when its HIP library is missing.

Modules:
  bf16            round-to-nearest-even fp32 -> bf16 helpers (numpy)
  echosparse_ref  numpy restatement of the EchoSparse kernel set (reference: echosparse/kernels/*.py)
  vsa_ref         numpy restatement of the VSA fine block-sparse attention and routers (reference: csrc/vsa,
                  tests/vsa_reference.py)
"""
