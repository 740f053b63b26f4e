"""Pieces shared by the pipeline integrations: the clock that tells the attention which denoising step, CFG branch
and layer a call belongs to and the 3D Morton token order (reference echosparse/models/common.py), and the
call routing every family uses: one patched dispatcher per diffusers module, one opaque custom op for all routed
calls, and the joint-sequence layout (video rows sparse, everything else a sink) of the families with a prefix or a
text suffix."""
import dataclasses
import functools
from typing import Optional

import torch

from ..attention import BK, dense_attention


class Clock:
    """(step, branch, layer) of the current attention call, driven by the pipeline's own calls (reference
    common.py:6-36): `scheduler.set_timesteps` starts a video (step 0, and every `on_reset` callback runs),
    `scheduler.step` closes a denoising step, each transformer forward opens the next branch (layer back to 0) and
    the attention dispatch advances `layer` after each self-attention call."""

    def __init__(self, pipe, on_reset=()):
        self.step, self.branch, self.layer = 0, -1, 0
        self._on_reset = list(on_reset)
        sched = pipe.scheduler
        self._wrap(sched, "set_timesteps", self._new_video)
        self._wrap(sched, "step", self._next_step)
        pipe.transformer.register_forward_pre_hook(self._new_branch)

    @staticmethod
    def _wrap(obj, name, before):
        inner = getattr(obj, name)

        @functools.wraps(inner)
        def wrapped(*args, **kwargs):
            before()
            return inner(*args, **kwargs)

        setattr(obj, name, wrapped)

    def _new_video(self):
        self.step, self.branch = 0, -1
        for fn in self._on_reset:
            fn()

    def _next_step(self):
        self.step += 1
        self.branch = -1

    def _new_branch(self, _module, _args):
        self.branch += 1
        self.layer = 0


def _spread3(v):
    """Bits 0..20 of each int64 in v moved to bits 0, 3, 6, .., 60 (the standard shift-and-mask bit spreading)."""
    v = v & 0x1FFFFF
    v = (v | (v << 32)) & 0x1F00000000FFFF
    v = (v | (v << 16)) & 0x1F0000FF0000FF
    v = (v | (v << 8)) & 0x100F00F00F00F00F
    v = (v | (v << 4)) & 0x10C30C30C30C30C3
    v = (v | (v << 2)) & 0x1249249249249249
    return v


def morton_code(t, y, x):
    """3D Morton (Z-order) code: bit i of x, y, t lands at bit 3i, 3i + 1, 3i + 2 (coordinates below 2^21)."""
    t, y, x = (c.to(torch.int64) for c in (t, y, x))
    return _spread3(x) | (_spread3(y) << 1) | (_spread3(t) << 2)


def morton_order(t, y, x):
    """Permutation that lists tokens with coordinates (t, y, x) in Morton order, and its inverse (reference
    common.py:39-45)."""
    perm = torch.argsort(morton_code(t, y, x))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel(), device=perm.device)
    return perm, inv


@functools.lru_cache(maxsize=8)
def grid_morton_order(frames, height, width, device):
    """Morton order of a raster-ordered (frames, height, width) token grid (reference common.py:48-53)."""
    t, y, x = torch.meshgrid(torch.arange(frames), torch.arange(height), torch.arange(width), indexing="ij")
    perm, inv = morton_order(t.reshape(-1), y.reshape(-1), x.reshape(-1))
    return perm.to(device), inv.to(device)


# ------------------------------------------------------------------------------------ attention call routing
# Every integration replaces the `dispatch_attention_fn` global of one diffusers transformer module (the function
# its attention processors call with [B, L, H, D] tensors). The replacement sorts each call into a numbered route or
# hands it back to diffusers; routed calls go through ONE opaque custom op, so a compiled transformer neither traces
# into the ctypes kernels nor specialises on the Python state of a route (clock, layouts).
_ROUTES = []


@torch.library.custom_op("echosparse_mi355x::routed_attention", mutates_args=())
def routed_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor],
                     route: int) -> torch.Tensor:
    return _ROUTES[route](q, k, v, mask)


@routed_attention.register_fake
def _(q, k, v, mask, route):
    return torch.empty_like(q)


def add_route(fn):
    """Register fn(q, k, v, mask) -> out as a route; returns its number."""
    _ROUTES.append(fn)
    return len(_ROUTES) - 1


@dataclasses.dataclass
class AttentionCall:
    """The arguments of one diffusers attention call that decide its route."""
    query: torch.Tensor
    key: torch.Tensor
    value: torch.Tensor
    mask: Optional[torch.Tensor]
    dropout_p: float
    is_causal: bool
    scale: Optional[float]
    parallel_config: object

    @property
    def plain(self):
        """Unmasked, no dropout, no causal mask, default scale, one device."""
        return (self.mask is None and self.dropout_p == 0.0 and not self.is_causal and self.scale is None
                and self.parallel_config is None)


def patch_dispatch(module, choose, pass_mask=False):
    """Replace module.dispatch_attention_fn. choose(AttentionCall) returns a route number, or None to keep the
    function the module had; routed calls get contiguous q / k / v (and the mask when pass_mask)."""
    original = module.dispatch_attention_fn

    def dispatch(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, scale=None, enable_gqa=False,
                 attention_kwargs=None, *, backend=None, parallel_config=None):
        route = choose(AttentionCall(query, key, value, attn_mask, dropout_p, is_causal, scale, parallel_config))
        if route is None:
            return original(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p, is_causal=is_causal,
                            scale=scale, enable_gqa=enable_gqa, attention_kwargs=attention_kwargs, backend=backend,
                            parallel_config=parallel_config)
        return routed_attention(query.contiguous(), key.contiguous(), value.contiguous(),
                                attn_mask if pass_mask else None, route)

    dispatch.original = original
    module.dispatch_attention_fn = dispatch
    return dispatch


def dense_route(q, k, v, _mask):
    """Route of calls that stay dense (cross-attention): the native dense kernel."""
    return dense_attention(q, k, v)


class SinkLayout:
    """A joint sequence whose first `valid` tokens are real (padding after them, output rows zero) and whose video
    span [start, start + n) runs through the sparse attention in the order `perm` (a permutation of 0..n-1).

    The sparse call sees [video in `perm` order | every other valid token]: the other tokens sit in the kv blocks
    from n // 64 on, which the attention computes exactly for every query tile (its `sink`), and only the first n
    query rows are used (`rows`). The other tokens' own query rows attend densely to every valid key, in the
    original order."""

    def __init__(self, start, perm, valid):
        n = perm.numel()
        dev = perm.device
        if start < 0 or start + n > valid:
            raise ValueError(f"video span [{start}, {start + n}) outside the {valid} valid tokens")
        self.start, self.n, self.valid = start, n, valid
        self.others = torch.cat([torch.arange(0, start, device=dev), torch.arange(start + n, valid, device=dev)])
        self.gather = torch.cat([perm + start, self.others])
        self.unperm = torch.argsort(perm)

    def __call__(self, attention, clock, q, k, v):
        qv, kv, vv = (x[:, :self.valid] for x in (q, k, v))
        o = attention(*(x.index_select(1, self.gather) for x in (qv, kv, vv)), clock.step, clock.branch,
                      clock.layer, sink=self.n // BK, rows=self.n)
        out = torch.zeros_like(q)
        out[:, self.start:self.start + self.n] = o[:, :self.n].index_select(1, self.unperm)
        if self.others.numel():
            rows = dense_attention(qv.index_select(1, self.others), kv.contiguous(), vv.contiguous())
            out.index_copy_(1, self.others, rows)
        clock.layer += 1
        return out
