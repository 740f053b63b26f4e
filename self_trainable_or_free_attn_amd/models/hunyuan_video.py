"""HunyuanVideo text-to-video (diffusers `HunyuanVideoPipeline`); behaviour of the reference's
echosparse/models/hunyuan_video.py.

The dual- and single-stream blocks attend over [video tokens | padded text tokens] with a key-padding mask; those
joint calls are routed to a `SinkLayout`: the padding is cropped, the video rows run sparse in Morton order with
the valid text tokens as a sink, and the text rows run dense over every valid key. Only the video rows enter the
sparse kernels (`rows`), since the text rows are computed densely anyway. Other calls (the token refiner) keep
diffusers' dispatcher. One transformer forward per step (embedded guidance).
"""
import torch

from .common import Clock, SinkLayout, add_route, grid_morton_order, patch_dispatch

TRANSFORMER_PREFIX = "HunyuanVideoTransformer"


class JointRoute:
    """The joint-attention route of one pipeline: the video grid from the transformer's input, the number of valid
    text tokens from the first joint call's mask (once per video: one host sync), and the layout built from both."""

    def __init__(self, pipe, attention):
        self.attention = attention
        self.clock = Clock(pipe, on_reset=[attention.reset, self._new_video])
        cfg = pipe.transformer.config
        self.patch = (cfg.patch_size_t, cfg.patch_size, cfg.patch_size)
        self.grid = None
        self.layout = None
        pipe.transformer.register_forward_pre_hook(self._read_grid, with_kwargs=True)

    @property
    def video_len(self):
        return 0 if self.grid is None else self.grid[0] * self.grid[1] * self.grid[2]

    def _new_video(self):
        self.layout = None

    def _read_grid(self, _module, args, kwargs):
        latents = kwargs.get("hidden_states", args[0] if args else None)
        grid = tuple(n // p for n, p in zip(latents.shape[-3:], self.patch))
        if grid != self.grid:
            self.grid, self.layout = grid, None

    def takes(self, call):
        """A joint call: masked self-attention over more tokens than the video has, nothing else unusual."""
        same = call.query.shape == call.key.shape == call.value.shape
        return (call.mask is not None and same and call.query.shape[1] > self.video_len
                and call.dropout_p == 0.0 and not call.is_causal and call.scale is None
                and call.parallel_config is None)

    def __call__(self, q, k, v, mask):
        if self.layout is None:
            # the mask is boolean (True = keep) or additive (0 = keep, -inf = drop); the text follows the video
            m = mask.reshape(q.shape[0], -1)[0, self.video_len:]
            text = int((m if m.dtype == torch.bool else m > -1.0).sum())
            perm, _ = grid_morton_order(*self.grid, q.device)
            self.layout = SinkLayout(0, perm, self.video_len + text)
        return self.layout(self.attention, self.clock, q, k, v)


def install(pipe, attention):
    """Route `pipe`'s joint attention calls (reference hunyuan_video.py:86-89); returns the route."""
    from diffusers.models.transformers import transformer_hunyuan_video
    joint = JointRoute(pipe, attention)
    number = add_route(joint)
    patch_dispatch(transformer_hunyuan_video, lambda call: number if joint.takes(call) else None, pass_mask=True)
    return joint
