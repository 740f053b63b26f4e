"""Wan2.1 text-to-video (diffusers `WanPipeline`); behaviour of the reference's echosparse/models/wan.py.

Routes: attention whose keys are as long as its queries (self-attention) runs through EchoSparseAttention with the
clock's (step, branch, layer); anything else (cross-attention over the text) through the native dense kernel. Wan
calls attention with no mask, dropout, causal mask or custom scale; other calls are refused.

Token order: the video tokens enter the first block in 3D Morton order and leave the last one in raster order, and
the rotary tables are permuted the same way, so every 64-token kv block is a compact space-time patch. The
permutation is made once per latent shape (cached) and applied by module hooks; no attention call reorders.
"""
from .common import Clock, add_route, dense_route, grid_morton_order, patch_dispatch

TRANSFORMER_PREFIX = "WanTransformer"


class MortonTokens:
    """Hooks that run every block of a Wan transformer on Morton-ordered tokens (reference wan.py:58-80 uses the
    same four points, which the transformer's structure dictates: its forward sees the latent grid, `rope` makes the
    per-token tables, blocks[0] takes the patch tokens and blocks[-1] hands them to the output head)."""

    def __init__(self, transformer):
        self.patch = tuple(transformer.config.patch_size)
        self.order = None
        transformer.register_forward_pre_hook(self._grid, with_kwargs=True)
        transformer.rope.register_forward_hook(self._tables)
        transformer.blocks[0].register_forward_pre_hook(self._enter)
        transformer.blocks[-1].register_forward_hook(self._leave)

    def _grid(self, _module, args, kwargs):
        latents = kwargs.get("hidden_states", args[0] if args else None)
        dims = [n // p for n, p in zip(latents.shape[-3:], self.patch)]
        self.order = grid_morton_order(*dims, latents.device)

    def _tables(self, _module, _args, tables):
        perm = self.order[0]
        return tuple(t.index_select(1, perm) for t in tables)

    def _enter(self, _module, args):
        return (args[0].index_select(1, self.order[0]), *args[1:])

    def _leave(self, _module, _args, out):
        return out.index_select(1, self.order[1])


def install(pipe, attention, morton=True):
    """Route `pipe`'s attention calls (reference wan.py:83-87); returns the clock."""
    from diffusers.models.transformers import transformer_wan
    clock = Clock(pipe, on_reset=[attention.reset])

    def self_attention(q, k, v, _mask):
        out = attention(q, k, v, clock.step, clock.branch, clock.layer)
        clock.layer += 1
        return out

    sparse, dense = add_route(self_attention), add_route(dense_route)

    def choose(call):
        if not (call.mask is None and call.dropout_p == 0.0 and not call.is_causal and call.scale is None):
            raise NotImplementedError("EchoSparse Wan attention: no mask, dropout, causal mask or custom scale")
        return sparse if call.key.shape[1] == call.query.shape[1] else dense

    patch_dispatch(transformer_wan, choose)
    if morton:
        MortonTokens(pipe.transformer)
    return clock
