"""MI355X-native block-sparse attention hot path of EchoSparse / VSA (reference package `echosparse`).

Public surface (mirrors the reference's):
  EchoSparseAttention       LSE-guided block-sparse self-attention (attention.py)
  backends                  device -> kernel set resolution ("auto" / "mi355x")
  kernels.gfx950            the kernel set (plugin interface), HIP kernels behind libechosparse_hip.so
"""
from .attention import EchoSparseAttention

__all__ = ["EchoSparseAttention"]
__version__ = "0.1.0"
