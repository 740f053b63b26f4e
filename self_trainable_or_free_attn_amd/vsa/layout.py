"""Real tokens <-> the block-padded layout the VSA operators take (reference echosparse/vsa/layout.py:1-128).

The permutation is the reference's, so tensors prepared for one package run on the other unchanged:
  * a 64-token block is one (tt, th, tw) tile of the (T, H, W) video grid (tt * th * tw = 64), tiles in raster
    order, valid tokens first, padding last;
  * inside a tile the order is sub-cube major: the tile splits into (st, sh, sw) sub-cubes of R = st * sh * sw
    tokens, sub-cubes in raster order, raster order inside each, so consecutive R tokens form one router group;
  * tiles cut by the grid boundary keep that order restricted to the tokens that exist, packed to the front.
`to_blocked` scatters real tokens into a zero buffer (padding = 0) and `from_blocked` gathers them back; both are
differentiable and give padding no gradient. `sequence_layout` is the 1-D form (blocks of 64 consecutive tokens).
Built with tensor index arithmetic on the host instead of per-token Python loops.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Tuple

import torch

SUBCUBE_FOR_R = {4: (1, 2, 2), 8: (2, 2, 2), 16: (1, 4, 4), 32: (2, 4, 4)}


@dataclass
class BlockLayout:
    shape: Tuple[int, ...]
    tile: Tuple[int, ...]
    sub: Tuple[int, ...]
    gather: torch.Tensor   # [NB * 64] raster index of the token in each padded slot, -1 for padding
    scatter: torch.Tensor  # [N] padded slot of each raster token
    blk_cnt: torch.Tensor  # [NB] int32 valid tokens per block

    @property
    def num_blocks(self) -> int:
        return self.blk_cnt.numel()

    @property
    def padded_len(self) -> int:
        return self.gather.numel()


def _tile_order(tile, sub):
    """Local (x, y, z) offsets of the 64 slots of a full tile, sub-cube major: [64, 3]."""
    tt, th, tw = tile
    st, sh, sw = sub
    outer = torch.cartesian_prod(torch.arange(tt // st), torch.arange(th // sh), torch.arange(tw // sw))
    inner = torch.cartesian_prod(torch.arange(st), torch.arange(sh), torch.arange(sw))
    step = torch.tensor([st, sh, sw])
    return (outer[:, None, :] * step + inner[None, :, :]).reshape(-1, 3)


def build_layout(shape, tile=(4, 4, 4), sub=None, R: int = 8, device="cpu") -> BlockLayout:
    T, H, W = shape
    tt, th, tw = tile
    assert tt * th * tw == 64, "hardware block must hold 64 tokens"
    sub = tuple(sub) if sub is not None else SUBCUBE_FOR_R[R]
    st, sh, sw = sub
    assert tt % st == 0 and th % sh == 0 and tw % sw == 0, "sub-cube must tile the block"
    local = _tile_order(tile, sub)                                                   # [64, 3]
    origins = torch.cartesian_prod(torch.arange(0, T, tt), torch.arange(0, H, th), torch.arange(0, W, tw))
    pos = origins[:, None, :] + local[None, :, :]                                    # [NB, 64, 3]
    inside = (pos[..., 0] < T) & (pos[..., 1] < H) & (pos[..., 2] < W)
    raster = (pos[..., 0] * H + pos[..., 1]) * W + pos[..., 2]
    # pack each block's existing tokens to the front, keeping the tile order (stable sort on "missing")
    order = torch.sort((~inside).to(torch.int8), dim=1, stable=True).indices
    packed = torch.gather(torch.where(inside, raster, torch.full_like(raster, -1)), 1, order)
    gather = packed.reshape(-1).to(torch.int64)
    cnt = inside.sum(1).to(torch.int32)
    scatter = torch.empty(T * H * W, dtype=torch.int64)
    slots = torch.nonzero(gather >= 0).squeeze(1)
    scatter[gather[slots]] = slots
    return BlockLayout(tuple(shape), tuple(tile), sub, gather.to(device), scatter.to(device), cnt.to(device))


def tail_block_counts(L_valid: int, device="cpu") -> torch.Tensor:
    """Valid-token count of each 64-token block when a sequence of L_valid tokens is cut into consecutive blocks:
    64 everywhere except the final block, which keeps the remainder."""
    starts = torch.arange(0, L_valid, 64, dtype=torch.int32)
    return (L_valid - starts).clamp(max=64).to(torch.int32).to(device)


def sequence_layout(n: int, device="cpu") -> BlockLayout:
    """Layout of a plain 1-D sequence: token i sits in slot i, the slots past n (the final block's padding) hold no
    token (gather index -1)."""
    cnt = tail_block_counts(n)
    slots = torch.arange(cnt.numel() * 64, dtype=torch.int64)
    gather = torch.where(slots < n, slots, torch.full_like(slots, -1))
    return BlockLayout((n,), (64,), (), gather.to(device), torch.arange(n, device=device), cnt.to(device))


def to_blocked(x: torch.Tensor, lay: BlockLayout) -> torch.Tensor:
    """Place the N real tokens of x [B, H, N, ...] into their block slots: [B, H, NB * 64, ...], zeros in the slots
    that hold no token."""
    out = x.new_zeros(*x.shape[:2], lay.padded_len, *x.shape[3:])
    return out.index_copy(2, lay.scatter, x)


def from_blocked(y: torch.Tensor, lay: BlockLayout) -> torch.Tensor:
    """Inverse of to_blocked: read every real token's slot of y [B, H, NB * 64, ...] back into the original token
    order, [B, H, N, ...]."""
    return y.index_select(2, lay.scatter)


def pad_tail(x: torch.Tensor, L_valid: int) -> torch.Tensor:
    """Extend x [B, H, L_valid, D] along the token axis with zero rows up to the next multiple of 64."""
    extra = -L_valid % 64
    if extra == 0:
        return x.contiguous()
    return torch.nn.functional.pad(x, (0, 0, 0, extra))
