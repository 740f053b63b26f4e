"""Wan2.1 text-to-video (diffusers `WanPipeline`), reference echosparse/models/wan.py.

Self-attention (query and key sequences of equal length) runs through EchoSparseAttention, cross-attention
(video queries over text keys) through the native dense kernel. The video tokens are put in 3D Morton order once,
before the first transformer block, together with the rotary tables, and put back after the last block, so every
64-token kv block is a compact space-time patch rather than a piece of one raster row.

Both attention calls are `torch.library.custom_op`s, so a compiled transformer treats them as opaque calls.
"""
import torch
from diffusers.models.transformers import transformer_wan

from ..attention import dense_attention
from .common import Clock, grid_morton_order

_self_attention_impl = None


@torch.library.custom_op("echosparse_mi355x::wan_self_attention", mutates_args=())
def _self_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    return _self_attention_impl(q, k, v)


@_self_attention.register_fake
def _(q, k, v):
    return torch.empty_like(q)


@torch.library.custom_op("echosparse_mi355x::wan_cross_attention", mutates_args=())
def _cross_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    return dense_attention(q, k, v)


@_cross_attention.register_fake
def _(q, k, v):
    return torch.empty_like(q)


def _dispatch(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, scale=None, enable_gqa=False,
              attention_kwargs=None, *, backend=None, parallel_config=None):
    """Replacement of diffusers' `dispatch_attention_fn` inside transformer_wan (reference wan.py:37-43)."""
    if attn_mask is not None or dropout_p != 0.0 or is_causal or scale is not None:
        raise NotImplementedError("EchoSparse Wan attention: no mask, dropout, causal mask or custom scale")
    q, k, v = query.contiguous(), key.contiguous(), value.contiguous()
    if k.shape[1] == q.shape[1]:
        return _self_attention(q, k, v)
    return _cross_attention(q, k, v)


class _SelfAttention:
    """Calls the attention with the clock's (step, branch, layer) and advances the layer."""

    def __init__(self, attention, clock):
        self.attention, self.clock = attention, clock

    def __call__(self, q, k, v):
        c = self.clock
        out = self.attention(q, k, v, c.step, c.branch, c.layer)
        c.layer += 1
        return out


class _MortonOrder:
    """Token order hooks (reference wan.py:58-80): the transformer's pre-hook reads the latent grid, the rotary
    module returns its tables in Morton order, block 0's pre-hook permutes the hidden states and the last block's
    hook restores raster order."""

    def __init__(self, transformer):
        self.patch = tuple(transformer.config.patch_size)
        self.perm = self.inv = None
        rope = transformer.rope.forward

        def rope_in_order(hidden_states):
            cos, sin = rope(hidden_states)
            return cos.index_select(1, self.perm), sin.index_select(1, self.perm)

        transformer.rope.forward = rope_in_order
        transformer.register_forward_pre_hook(self._set_grid, with_kwargs=True)
        transformer.blocks[0].register_forward_pre_hook(self._to_morton)
        transformer.blocks[-1].register_forward_hook(self._to_raster)

    def _set_grid(self, _module, args, kwargs):
        x = kwargs["hidden_states"] if "hidden_states" in kwargs else args[0]
        f, h, w = x.shape[2:]
        pt, ph, pw = self.patch
        self.perm, self.inv = grid_morton_order(f // pt, h // ph, w // pw, x.device)

    def _to_morton(self, _module, args):
        return (args[0].index_select(1, self.perm),) + tuple(args[1:])

    def _to_raster(self, _module, _args, out):
        return out.index_select(1, self.inv)


def enable(pipe, attention, morton=True):
    """Install the Wan hooks on `pipe` (reference wan.py:83-87)."""
    global _self_attention_impl
    clock = Clock(pipe, on_reset=[attention.reset])
    _self_attention_impl = _SelfAttention(attention, clock)
    transformer_wan.dispatch_attention_fn = _dispatch
    if morton:
        _MortonOrder(pipe.transformer)
    return clock
