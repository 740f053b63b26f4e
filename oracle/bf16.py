"""bf16 / fp16 helpers for the CPU oracle (test infrastructure only, see oracle/__init__.py).

16-bit values are held in float32 arrays; `round_bf16` applies IEEE round-to-nearest-even to 8 mantissa bits, the
conversion the reference's `.to(tl.bfloat16)` / `.to(torch.bfloat16)` performs; `round_f16` is numpy's IEEE binary16
conversion (round to nearest even, overflow to inf), the reference's `.to(torch.float16)` / `__float2half`. Both are
pinned by tests against torch's own conversions.
"""
import numpy as np


def round_bf16(x):
    """float32 array -> float32 array holding the nearest bf16 values (ties to even; NaN stays NaN)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out).astype(np.float32)


def to_bf16_bits(x):
    """float32 array -> uint16 bf16 bit patterns (round to nearest even)."""
    return (round_bf16(x).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(b):
    """uint16 bf16 bit patterns -> float32 array."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_f16(x):
    """float32 array -> float32 array holding the nearest fp16 values (ties to even, overflow to inf)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
