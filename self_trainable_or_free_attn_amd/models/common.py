"""Pieces shared by the pipeline integrations (reference echosparse/models/common.py): the clock that tells the
attention which denoising step, CFG branch and layer a call belongs to, and the 3D Morton token order."""
import functools

import torch


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
