"""MI355X-native block-sparse attention hot path of EchoSparse / VSA (reference package `echosparse`).

Public surface (mirrors the reference's):
  EchoSparseAttention       LSE-guided block-sparse self-attention (attention.py)
  enable, PRESETS           route a diffusers pipeline's self-attention through it (models/)
  backends                  device -> kernel set resolution ("auto" / "mi355x")
  kernels.gfx950            the kernel set (plugin interface), HIP kernels behind libechosparse_hip.so
"""
from .attention import EchoSparseAttention
from .models import PRESETS, enable

__all__ = ["EchoSparseAttention", "PRESETS", "enable"]
__version__ = "0.1.0"
