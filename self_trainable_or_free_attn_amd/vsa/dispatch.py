"""Which generic fine-backward variant an operator call records (reference echosparse/vsa/dispatch.py:1-53).

The variants name how the reference computes dQ: 0 float2 atomics, 1 one-float atomics, 2 a separate q->kv pass
without atomics. This build has one deterministic dQ pass (the Q-owner kernel) and runs it for every variant, so the
choice changes no number; it is still resolved with the reference's precedence (per-call argument, then
ops.set_bwd_variant, then the ECHOSPARSE_VSA_BWD_VARIANT environment variable, then the automatic rule) and exposed
on ``o.grad_fn`` so code that inspects it keeps working. The automatic rule here always answers 2, the variant that
matches what runs. No torch import, so CPU checks can load this module alone.
"""
import os
from typing import Optional, Tuple

BWD_VARIANTS = (0, 1, 2)
ENV_NAME = "ECHOSPARSE_VSA_BWD_VARIANT"


def check_bwd_variant(v, what: str) -> int:
    if v not in BWD_VARIANTS:
        raise ValueError(f"{what} must be one of {BWD_VARIANTS}, got {v!r}")
    return int(v)


def auto_bwd_variant(B: int, H: int, L: int, D: int, gpu_major: int) -> int:
    """MI355X: the atomics-free dQ pass is the only one built."""
    return 2


def _from_environment(environ):
    """The variant named by ECHOSPARSE_VSA_BWD_VARIANT, None when unset; a value that is not an int is refused with
    the same message as an out-of-range one."""
    raw = environ.get(ENV_NAME)
    if raw is None:
        return None
    try:
        return int(raw)
    except ValueError:
        raise ValueError(f"{ENV_NAME} must be one of {BWD_VARIANTS}, got {raw!r}") from None


def select_bwd_variant(B: int, H: int, L: int, D: int, gpu_major: int, call: Optional[int] = None,
                       override: Optional[int] = None, environ=os.environ) -> Tuple[int, str]:
    """(variant, source) from the first of: the per-call argument, ops.set_bwd_variant, the environment variable,
    the automatic rule; source is "call", "set_bwd_variant", "environment" or "auto"."""
    candidates = (("call", "bwd_variant", lambda: call), ("set_bwd_variant", "set_bwd_variant", lambda: override),
                  ("environment", ENV_NAME, lambda: _from_environment(environ)))
    for source, what, value in candidates:
        v = value()
        if v is not None:
            return check_bwd_variant(v, what), source
    return auto_bwd_variant(B, H, L, D, gpu_major), "auto"
