"""MI355X (gfx950) kernel set: the function set of the reference's `echosparse.kernels.sm90` / `sm120` modules
(the plugin interface `echosparse.attention` calls), each a thin wrapper over one C-ABI call of
libechosparse_hip.so (include/echosparse_hip.h).

Same quantities and units as the reference sets: q / k / v are (L, H, D) bf16 with D = 128; 128-row query tiles,
64-token kv blocks; the previous step's log2 LSE as a fixed softmax offset ((nq * 128, H) float32, 1e30 past L);
block masses summed over the tile's rows into (H, nq, nb) float32. Every function writes in place into caller
tensors and returns None, like the reference's.
"""
import math

import torch

from .. import _lib

BM = 128
BK = 64
LOG2E = 1.4426950408889634


def _cdiv(a, b):
    return -(-a // b)


def _check_qkv(q, *others):
    L, H, D = q.shape
    assert D == 128 and q.dtype == torch.bfloat16, "q must be (L, H, 128) bf16"
    for x in (q, *others):
        assert x.is_cuda and x.is_contiguous(), "tensors must be contiguous GPU tensors"
    return L, H, D


def block_means(k, v, k_mean, v_mean):
    """Mean key and value of every 64-token block: (L, H, D) -> (nb, H, D). Reference triton_ops.py:37-40."""
    L, H, D = _check_qkv(k, v, k_mean, v_mean)
    _lib.call("es_block_means", k, v, k_mean, v_mean, L, H, D)


def select_blocks(mass, keep_prev, scale_exact, scale_skip, keep, counts, blocks, flags, skip_bits, refine, k, r, L,
                  sink=1 << 30):
    """Top-k blocks of every (query tile, head) by block probability, plus the forced ones; the refine list (the
    top-r skipped blocks) and the bit mask of blocks the block-mean compensation leaves out. Reference
    triton_ops.py:108-119 (bit-exact)."""
    H, nq, nb = mass.shape
    nbp = 1 << (nb - 1).bit_length()
    assert refine.shape[-1] >= r and refine.shape[-1] <= nbp
    assert blocks.shape[-1] == nb, "blocks must be (nq, H, nb)"
    _lib.call("es_select_blocks", mass, keep_prev, scale_exact, scale_skip, keep, counts, blocks, flags, skip_bits,
              skip_bits.shape[-1], refine, refine.shape[-1], int(k), int(r), int(L), H, int(min(sink, 2**31 - 1)))


def estimate_skipped(q, k_mean, keep, offset, lse, mass, scale_exact, scale_skip):
    """Mass estimates of the skipped blocks for the next step's selection, and the per-tile scales. Reference
    triton_ops.py:170-177 (sm120.py:240-250 computes the same values)."""
    L, H, D = _check_qkv(q, k_mean)
    _lib.call("es_estimate_skipped", q, k_mean, keep, offset, lse, mass, scale_exact, scale_skip, L, H, D)


def full_step_scales(offset, lse, scale_exact, scale_skip, L):
    """Map scales after a step that computed every block; resets the padding rows of `lse` to 1e30. Reference
    triton_ops.py:196-199."""
    H = scale_exact.shape[0]
    _lib.call("es_full_step_scales", offset, lse, scale_exact, scale_skip, int(L), H)


def exact_fallback(q, k, v, out, counts, blocks, lse, flags):
    """Online-softmax attention over the block list, for the tiles whose fixed offset was too far off. Reference
    sm120.py:176-180."""
    L, H, D = _check_qkv(q, k, v, out)
    _lib.call("es_exact_fallback", q, k, v, out, counts, blocks, blocks.shape[-1], lse, flags, L, H, D)


def compensate_fallback(q, k_mean, v_mean, keep, lse, out, flags):
    """Block-mean compensation of the skipped blocks for the fallback tiles, in place on `out` and `lse`.
    Reference triton_ops.py:285-295."""
    L, H, D = _check_qkv(q, k_mean, v_mean, out)
    _lib.call("es_compensate_fallback", q, k_mean, v_mean, keep, lse, out, flags, L, H, D)


def block_attention(q, k, v, out, counts, blocks, offset, lse, flags, mass=None, threshold=60.0):
    """Exact attention over a list of 64-token kv blocks with a fixed offset, plus per-block masses. Reference
    sm90.py:118-127."""
    L, H, D = _check_qkv(q, k, v, out)
    _lib.call("es_block_attention", q, k, v, out, counts, blocks, blocks.shape[-1], offset, lse, flags, mass,
              float(threshold), L, H, D)


def launched_tiles(out, lse, flags, offset, rows):
    """Query tiles to launch: the caller only uses query rows < rows (it overwrites the others), so the tiles past
    them are not launched; their output is zero, their LSE the offset and their flag 0. Reference
    sm120.py:111-120."""
    nq = _cdiv(out.shape[0], BM)
    tiles = nq if rows is None else min(nq, _cdiv(rows, BM))
    if tiles < nq:
        flags[tiles:].zero_()
        out[tiles * BM:].zero_()
        lse[tiles * BM:].copy_(offset[tiles * BM:])
    return tiles


def sparse_attention(q, k, v, k_mean, v_mean, means, mean_counts, out, counts, blocks, offset, lse, flags, refine,
                     refine_counts, k_rep, v_rep, log_counts, mass=None, threshold=60.0, rows=None):
    """Listed blocks exactly, the listed mean blocks through block means and the listed refined blocks through four
    representatives each, in one softmax at the fixed offset. The lists are `rebuild_plan`'s; `rows`: see
    `launched_tiles`. Reference sm120.py:123-140 / sm90.py:130-144."""
    L, H, D = _check_qkv(q, k, v, out, k_mean, v_mean, k_rep, v_rep)
    tiles = launched_tiles(out, lse, flags, offset, rows)
    if tiles == 0:
        return
    _lib.call("es_sparse_attention", q, k, v, k_mean, v_mean, means, mean_counts, out, counts, blocks,
              blocks.shape[-1], offset, lse, flags, refine, refine_counts, refine.shape[-1], k_rep, v_rep,
              log_counts, mass, float(threshold), tiles, L, H, D)


def pack_plan(keep, exact_bits):
    """Bit mask of the exactly computed blocks: keep (H, nq, nb) uint8 -> exact_bits (H, nq, NW) int32. Reference
    sm120.py:268-273."""
    H, nq, nb = keep.shape
    _lib.call("es_pack_plan", keep, exact_bits, exact_bits.shape[-1], H, nq, nb)


def rebuild_plan(exact_bits, skip_bits, keep, counts, blocks, refine, refine_counts, means, mean_counts):
    """keep mask, sorted block list, refine list (padded with nb) and sorted list of the blocks left to their means,
    with the lengths of the last two, from the two bit masks of a plan. Reference sm120.py:299-305."""
    H, nq, nb = keep.shape
    assert blocks.shape[-1] == nb and means.shape[-1] == nb
    _lib.call("es_rebuild_plan", exact_bits, skip_bits, exact_bits.shape[-1], keep, counts, blocks, refine,
              refine_counts, refine.shape[-1], means, mean_counts, H, nq, nb)


def dense_attention(q, k, v):
    """Dense attention over all keys: returns (out (L, H, D) bf16, lse (nq * 128, H) float32 in log2 units with
    1e30 past L) -- the replacement of the FlashAttention-4 call that seeds the offsets."""
    L, H, D = _check_qkv(q, k, v)
    out = torch.empty_like(q)
    lse = torch.empty(_cdiv(L, BM) * BM, H, device=q.device, dtype=torch.float32)
    _lib.call("es_dense_attention", q, k, v, out, lse, L, H, D)
    return out, lse


def dense_attention_kv(q, k, v):
    """Dense attention of q (Lq, H, D) over k / v (Lk, H, D), any Lk: returns (out (Lq, H, D) bf16, lse (nq * 128,
    H) float32 log2 with 1e30 past Lq). The cross-attention / text-row calls of the pipeline integrations."""
    Lq, H, D = _check_qkv(q, k, v)
    Lk = k.shape[0]
    assert k.shape == v.shape == (Lk, H, D), "k and v must be (Lk, H, 128) with q's heads"
    out = torch.empty_like(q)
    lse = torch.empty(_cdiv(Lq, BM) * BM, H, device=q.device, dtype=torch.float32)
    _lib.call("es_dense_attention_kv", q, k, v, out, lse, Lq, Lk, H, D)
    return out, lse


class Representatives:
    """Four representatives per 64-token kv block, clustered in the query metric; buffers are reused across calls.
    Reference representatives.py:131-166 (same outputs: k / v (H, (nb + 1) * 4, D) bf16 and log_counts
    (H, (nb + 1) * 4) float32, with the empty sentinel block nb)."""

    def __init__(self, L, H, D, device, iters=6):
        nb = _cdiv(L, BK)
        assert nb >= 64, "needs at least 64 kv blocks (4096 tokens)"
        self.L, self.H, self.D, self.nb, self.iters = L, H, D, nb, iters
        nb4 = (nb + 1) * 4
        self.k = torch.zeros(H, nb4, D, device=device, dtype=torch.bfloat16)
        self.v = torch.zeros(H, nb4, D, device=device, dtype=torch.bfloat16)
        self.log_counts = torch.full((H, nb4), -math.inf, device=device)
        self._ws = torch.empty(_lib.workspace_bytes(L, H, D), device=device, dtype=torch.uint8)

    def build(self, q, k, v, k_mean=None, v_mean=None):
        """Representatives of every block; given k_mean / v_mean (nb, H, D), also the block means."""
        L, H, D = _check_qkv(q, k, v)
        assert (L, H, D) == (self.L, self.H, self.D)
        _lib.call("es_representatives", q, k, v, self.k, self.v, self.log_counts, k_mean, v_mean, self._ws,
                  self._ws.numel(), int(self.iters), L, H, D)
