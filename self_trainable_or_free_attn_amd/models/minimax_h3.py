"""MiniMax-H3 text-to-video-and-audio (the minimax-h3 branch of diffusers, `ModularPipeline`); behaviour of the
reference's echosparse/models/minimax_h3.py on the H100 / B200 layout.

H3 attends over one packed, unmasked sequence [text | conditioning | audio | target video]. Calls over the whole
packed sequence are routed to a `SinkLayout`: the target-video tail runs sparse in the Morton order of its rotary
(t, h, w) coordinates, everything before it is the sink and its rows run dense. Calls of other lengths (text rows
before packing) keep diffusers' dispatcher. Guidance-distilled checkpoint: one transformer forward per step.

The reference's RTX 5090-only layout (the model's index arguments remapped once per forward, its own rotary kernel)
is not part of this backend.
"""
import torch

from .common import Clock, SinkLayout, add_route, morton_order, patch_dispatch

TRANSFORMER_PREFIX = "MiniMaxH3"


def target_video_start(video_indices):
    """Index into `video_indices` (ascending token positions of every video) where its last run of consecutive
    positions, the target video, begins: video_indices[i] - i is non-decreasing and constant exactly on each run."""
    n = video_indices.numel()
    shift = video_indices - torch.arange(n, device=video_indices.device)
    return int((shift < shift[-1]).sum())


def axis_ranks(coords):
    """Each column of integer coordinates (N, 3) replaced by its dense rank among that column's values (the rotary
    time axis is strided)."""
    cols = []
    for a in range(coords.shape[1]):
        c = coords[:, a].contiguous()
        cols.append(torch.searchsorted(torch.unique(c), c).long())
    return cols


def packed_layout(position_ids, video_indices):
    """SinkLayout of a packed H3 sequence (reference minimax_h3.py:29-42 finds the same split and order)."""
    L = int(position_ids.shape[0])
    vs = int(video_indices[target_video_start(video_indices)].item())       # one host sync per layout
    if int(video_indices[-1].item()) != L - 1:
        raise ValueError("MiniMax-H3 layout: the target video must be the tail of the packed sequence")
    perm, _ = morton_order(*axis_ranks(position_ids[vs:]))
    return SinkLayout(vs, perm, L)


class PackedRoute:
    """The packed-sequence route of one pipeline; the layout is rebuilt when the sequence length changes."""

    def __init__(self, pipe, attention):
        self.attention = attention
        self.clock = Clock(pipe, on_reset=[attention.reset])
        self.layout = None
        pipe.transformer.register_forward_pre_hook(self._read_layout, with_kwargs=True)

    def _read_layout(self, _module, _args, kwargs):
        pos = kwargs["position_ids"]
        if self.layout is None or pos.shape[0] != self.layout.valid:
            self.layout = packed_layout(pos, kwargs["video_indices"])

    def choose(self, call, number):
        if self.layout is None or call.query.shape[1] != self.layout.valid:
            return None
        if not call.plain:
            raise NotImplementedError("EchoSparse MiniMax-H3 attention: no mask, dropout, causal mask, custom scale "
                                      "or parallel config")
        return number

    def __call__(self, q, k, v, _mask):
        return self.layout(self.attention, self.clock, q, k, v)


def install(pipe, attention):
    """Route `pipe`'s packed-sequence attention calls (reference minimax_h3.py:119-122); returns the route."""
    from diffusers.models.transformers import transformer_minimax_h3
    packed = PackedRoute(pipe, attention)
    number = add_route(packed)
    patch_dispatch(transformer_minimax_h3, lambda call: packed.choose(call, number))
    return packed
