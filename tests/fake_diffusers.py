"""Stand-ins for the three diffusers transformer modules the pipeline integrations patch, and small transformers
that call attention the way those modules do (diffusers is not installed here). Each fake module holds a
`dispatch_attention_fn` that the fake transformers look up at call time, as diffusers' modules do, so the
integration's replacement is what runs. The default dispatcher is plain (masked) scaled-dot-product attention.

Shapes follow diffusers: attention tensors are [B, L, H, D]; Wan / HunyuanVideo latents [B, C, F, H, W] with
patch sizes from `config`; MiniMax-H3 takes one packed sequence plus `position_ids` (L, 3) and `video_indices`."""
import sys
import types

import torch
import torch.nn.functional as F

NAMES = ("transformer_wan", "transformer_hunyuan_video", "transformer_minimax_h3")


def sdpa(q, k, v, attn_mask=None):
    """[B, L, H, D] attention in the inputs' dtype; attn_mask boolean [B, 1, 1, Lk] (True = keep)."""
    out = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                         attn_mask=attn_mask)
    return out.transpose(1, 2)


def default_dispatch(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, scale=None,
                     enable_gqa=False, attention_kwargs=None, *, backend=None, parallel_config=None):
    default_dispatch.calls += 1
    return sdpa(query, key, value, attn_mask)


default_dispatch.calls = 0


def install():
    """Put the fake `diffusers.models.transformers.*` modules into sys.modules (once) and return them by name."""
    root = sys.modules.get("diffusers")
    if root is None or not getattr(root, "_is_fake", False):
        root = types.ModuleType("diffusers")
        root._is_fake = True
        models = types.ModuleType("diffusers.models")
        transformers = types.ModuleType("diffusers.models.transformers")
        root.models, models.transformers = models, transformers
        sys.modules.update({"diffusers": root, "diffusers.models": models,
                            "diffusers.models.transformers": transformers})
        for name in NAMES:
            mod = types.ModuleType(f"diffusers.models.transformers.{name}")
            mod.dispatch_attention_fn = default_dispatch
            setattr(transformers, name, mod)
            sys.modules[mod.__name__] = mod
    return {name: sys.modules[f"diffusers.models.transformers.{name}"] for name in NAMES}


class Scheduler:
    def __init__(self):
        self.timesteps = []

    def set_timesteps(self, n):
        self.timesteps = list(range(n))

    def step(self, *_):
        return None


class Pipe:
    def __init__(self, transformer):
        self.transformer = transformer
        self.scheduler = Scheduler()


def _rotary(x, cos, sin):
    x1, x2 = x[..., 0::2], x[..., 1::2]
    rot = torch.stack((-x2, x1), dim=-1).flatten(-2)
    return x * cos + rot * sin


class _Rope(torch.nn.Module):
    """Per-token rotary tables (1, L, 1, D) of the raster-ordered patch grid."""

    def __init__(self, patch, D):
        super().__init__()
        self.patch, self.D = patch, D

    def forward(self, hidden_states):
        f, h, w = (n // p for n, p in zip(hidden_states.shape[2:], self.patch))
        pos = torch.arange(f * h * w, device=hidden_states.device, dtype=torch.float32)
        freq = 1.0 / (1000.0 ** (torch.arange(self.D // 2, device=pos.device, dtype=torch.float32) / (self.D // 2)))
        ang = (pos[:, None] * freq[None]).repeat_interleave(2, dim=1)
        return ang.cos()[None, :, None], ang.sin()[None, :, None]


def _patchify(x, patch):
    B, C, f, h, w = x.shape
    pt, ph, pw = patch
    x = x.reshape(B, C, f // pt, pt, h // ph, ph, w // pw, pw)
    return x.permute(0, 2, 4, 6, 1, 3, 5, 7).reshape(B, (f // pt) * (h // ph) * (w // pw), C * pt * ph * pw)


class _WanBlock(torch.nn.Module):
    def __init__(self, mod, dim, H, D):
        super().__init__()
        self.mod, self.H, self.D = mod, H, D
        self.qkv = torch.nn.Linear(dim, 3 * H * D, bias=False)
        self.q2 = torch.nn.Linear(dim, H * D, bias=False)
        self.kv2 = torch.nn.Linear(dim, 2 * H * D, bias=False)
        self.out = torch.nn.Linear(H * D, dim, bias=False)

    def forward(self, x, enc, rope):
        B, L, _ = x.shape
        q, k, v = self.qkv(x).reshape(B, L, 3, self.H, self.D).unbind(2)
        cos, sin = rope
        q, k = _rotary(q, cos, sin).to(x.dtype), _rotary(k, cos, sin).to(x.dtype)
        o = self.mod.dispatch_attention_fn(q, k, v)
        q2 = self.q2(x).reshape(B, L, self.H, self.D)
        k2, v2 = self.kv2(enc).reshape(B, enc.shape[1], 2, self.H, self.D).unbind(2)
        o2 = self.mod.dispatch_attention_fn(q2, k2, v2)
        return x + self.out((o + o2).reshape(B, L, -1))


class WanTransformer3DModel(torch.nn.Module):
    """Wan-like: patchify, rotary tables from `rope`, blocks of self- plus cross-attention."""

    def __init__(self, mod, C=4, H=2, D=128, depth=2, patch=(1, 2, 2)):
        super().__init__()
        self.config = types.SimpleNamespace(patch_size=patch)
        dim = 64
        self.embed = torch.nn.Linear(C * patch[0] * patch[1] * patch[2], dim, bias=False)
        self.rope = _Rope(patch, D)
        self.blocks = torch.nn.ModuleList(_WanBlock(mod, dim, H, D) for _ in range(depth))

    def forward(self, hidden_states, encoder_hidden_states):
        rope = self.rope(hidden_states)
        x = self.embed(_patchify(hidden_states, self.config.patch_size))
        for blk in self.blocks:
            x = blk(x, encoder_hidden_states, rope)
        return x


class HunyuanVideoTransformer3DModel(torch.nn.Module):
    """HunyuanVideo-like: [video | padded text] joint attention with a boolean key-padding mask, plus one
    unmasked text-only ("refiner") attention call first."""

    def __init__(self, mod, C=4, H=2, D=128, depth=2, patch_t=1, patch=2):
        super().__init__()
        self.mod, self.H, self.D = mod, H, D
        self.config = types.SimpleNamespace(patch_size_t=patch_t, patch_size=patch)
        dim = 64
        self.embed = torch.nn.Linear(C * patch_t * patch * patch, dim, bias=False)
        self.qkv = torch.nn.ModuleList(torch.nn.Linear(dim, 3 * H * D, bias=False) for _ in range(depth))
        self.out = torch.nn.ModuleList(torch.nn.Linear(H * D, dim, bias=False) for _ in range(depth))

    def forward(self, hidden_states, encoder_hidden_states, encoder_attention_mask):
        p = self.config.patch_size
        x = self.embed(_patchify(hidden_states, (self.config.patch_size_t, p, p)))
        B, vl, _ = x.shape
        T = encoder_hidden_states.shape[1]
        t = encoder_hidden_states
        tq, tk, tv = self.qkv[0](t).reshape(B, T, 3, self.H, self.D).unbind(2)
        t = t + self.out[0](self.mod.dispatch_attention_fn(tq, tk, tv).reshape(B, T, -1))  # refiner
        joint = torch.cat([x, t], dim=1)
        keep = torch.cat([torch.ones(B, vl, dtype=torch.bool, device=x.device), encoder_attention_mask], 1)
        mask = keep[:, None, None, :]
        for qkv, out in zip(self.qkv, self.out):
            q, k, v = qkv(joint).reshape(B, vl + T, 3, self.H, self.D).unbind(2)
            joint = joint + out(self.mod.dispatch_attention_fn(q, k, v, attn_mask=mask).reshape(B, vl + T, -1))
        return joint


class MiniMaxH3Transformer(torch.nn.Module):
    """MiniMax-H3-like: one packed sequence, unmasked attention over it, `position_ids` and `video_indices` as
    keyword arguments, plus one shorter attention call (text rows before packing)."""

    def __init__(self, mod, H=2, D=128, depth=2):
        super().__init__()
        self.mod, self.H, self.D = mod, H, D
        dim = 64
        self.qkv = torch.nn.ModuleList(torch.nn.Linear(dim, 3 * H * D, bias=False) for _ in range(depth))
        self.out = torch.nn.ModuleList(torch.nn.Linear(H * D, dim, bias=False) for _ in range(depth))

    def forward(self, hidden_states, *, position_ids, video_indices):
        x = hidden_states
        B, L, _ = x.shape
        head = x[:, :7]
        q, k, v = self.qkv[0](head).reshape(B, 7, 3, self.H, self.D).unbind(2)
        self.mod.dispatch_attention_fn(q, k, v)
        for qkv, out in zip(self.qkv, self.out):
            q, k, v = qkv(x).reshape(B, L, 3, self.H, self.D).unbind(2)
            x = x + out(self.mod.dispatch_attention_fn(q, k, v).reshape(B, L, -1))
        return x


def h3_positions(prefix, frames, height, width, device=None):
    """position_ids (prefix + f*h*w, 3) with a strided time axis for the target video, and video_indices that
    list a short conditioning-video run inside the prefix, then the target video."""
    t, y, x = torch.meshgrid(torch.arange(frames) * 4, torch.arange(height), torch.arange(width), indexing="ij")
    vid = torch.stack([t.reshape(-1), y.reshape(-1), x.reshape(-1)], 1)
    pre = torch.stack([torch.arange(prefix)] * 3, 1)
    pos = torch.cat([pre, vid]).to(device)
    vi = torch.cat([torch.arange(2, min(prefix, 9)), torch.arange(prefix, prefix + vid.shape[0])]).to(device)
    return pos, vi
