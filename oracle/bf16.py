"""bf16 helpers for the CPU oracle (test infrastructure only, see oracle/__init__.py).

bf16 values are held in float32 arrays; `round_bf16` applies IEEE round-to-nearest-even to 8 mantissa bits, the
conversion the reference's `.to(tl.bfloat16)` / `.to(torch.bfloat16)` performs. Pinned by tests against
torch's own float32 -> bfloat16 conversion.
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
