"""MiniMax-H3 text-to-video-and-audio (the minimax-h3 branch of diffusers, `ModularPipeline`), reference
echosparse/models/minimax_h3.py.

H3 attends over one packed, unmasked sequence [text | conditioning | audio | target video]. Everything before the
target-video tail is the prefix: its keys are a sink every query tile computes exactly, and its own query rows run
through the native dense kernel. The target-video rows run through EchoSparseAttention in Morton order, taken from
their rotary (t, h, w) coordinates. Attention calls of other lengths (text-only rows before packing) keep
diffusers' dispatcher. Guidance-distilled checkpoint: one transformer forward per step.

Token layout: each layer gathers q / k / v into [target video in Morton order | prefix] and scatters the output
back (the reference's H100 / B200 layout, minimax_h3.py:87-92). The reference's RTX 5090-only alternative, which
remaps the model's index arguments once per forward and ships its own rotary kernel, is not part of this backend.
"""
import torch
from diffusers.models.transformers import transformer_minimax_h3 as th3

from ..attention import BK, dense_attention
from .common import Clock, morton_order

_impl = None
_original_dispatch = th3.dispatch_attention_fn


class _Layout:
    """Where the target video sits in the packed sequence and its Morton order (reference minimax_h3.py:29-42)."""

    def __init__(self, position_ids, video_indices):
        L = int(position_ids.shape[0])
        # the target video is the last run of consecutive entries of video_indices (one host sync per layout)
        gaps = (video_indices[1:] - video_indices[:-1] != 1).nonzero()
        first = int(gaps[-1].item()) + 1 if gaps.numel() else 0
        vs = int(video_indices[first].item())
        # rotary coordinates need not be consecutive integers (t is strided): rank each axis first
        t, y, x = (torch.unique(position_ids[vs:, a], return_inverse=True)[1].long() for a in range(3))
        perm, _ = morton_order(t, y, x)
        self.L, self.video, self.video_start = L, L - vs, vs
        self.positions = position_ids.clone()
        # packed position p holds original token packed_to_original[p]: [video in Morton order | prefix]
        self.packed_to_original = torch.cat([perm + vs, torch.arange(vs, device=perm.device)])
        self.original_to_packed = torch.argsort(self.packed_to_original)


class _PackedAttention:
    """The packed-sequence attention of one pipeline (reference minimax_h3.py:52-98, non-packed layout)."""

    def __init__(self, pipe, attention):
        self.attention = attention
        self.clock = Clock(pipe, on_reset=[attention.reset])
        self.layout = None
        pipe.transformer.register_forward_pre_hook(self._set_layout, with_kwargs=True)

    @property
    def seq_len(self):
        return None if self.layout is None else self.layout.L

    def _set_layout(self, _module, args, kwargs):
        pos = kwargs["position_ids"]
        # a new layout when the sequence length changes (the reference's per-layer-gather layout does the same)
        if self.layout is None or pos.shape[0] != self.layout.L:
            self.layout = _Layout(pos, kwargs["video_indices"])

    def __call__(self, q, k, v):
        lay = self.layout
        nv, vs = lay.video, lay.video_start
        c = self.clock
        o = self.attention(*(x.index_select(1, lay.packed_to_original) for x in (q, k, v)), c.step, c.branch,
                           c.layer, sink=nv // BK, rows=nv)
        out = torch.empty_like(q)
        out[:, vs:] = o[:, :nv].index_select(1, lay.original_to_packed[vs:])
        out[:, :vs] = dense_attention(q[:, :vs].contiguous(), k, v)
        c.layer += 1
        return out


def _dispatch(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, scale=None, enable_gqa=False,
              attention_kwargs=None, *, backend=None, parallel_config=None):
    """Replacement of diffusers' `dispatch_attention_fn` inside transformer_minimax_h3 (reference
    minimax_h3.py:101-109)."""
    if query.shape[1] != _impl.seq_len:
        return _original_dispatch(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p, is_causal=is_causal,
                                  scale=scale, enable_gqa=enable_gqa, attention_kwargs=attention_kwargs,
                                  backend=backend, parallel_config=parallel_config)
    if attn_mask is not None or dropout_p != 0.0 or is_causal or scale is not None or parallel_config is not None:
        raise NotImplementedError("EchoSparse MiniMax-H3 attention: no mask, dropout, causal mask, custom scale or "
                                  "parallel config")
    return _impl(query.contiguous(), key.contiguous(), value.contiguous())


def enable(pipe, attention):
    """Install the MiniMax-H3 hooks on `pipe` (reference minimax_h3.py:119-122)."""
    global _impl
    _impl = _PackedAttention(pipe, attention)
    th3.dispatch_attention_fn = _dispatch
    return _impl
