"""Pipeline integrations (reference echosparse/models/__init__.py): `enable(pipe)` routes a diffusers video
pipeline's self-attention through EchoSparseAttention on MI355X.

    wan              diffusers WanPipeline (Wan2.1): self-attention sparse, cross-attention dense
    hunyuan_video    diffusers HunyuanVideoPipeline: video rows sparse with the text tokens as a sink
    minimax_h3       the minimax-h3 branch of diffusers: target-video rows sparse, the prefix as a sink

diffusers is imported only by the family module `enable` picks, so the package imports without it.
"""
from ..attention import EchoSparseAttention

# The settings of the reference's reported results (reference models/__init__.py:5-10), kept as published.
PRESETS = {
    "wan": dict(density=0.10, dense_steps=10, dense_layers=(0,)),
    "hunyuan_video": dict(density=0.10, dense_steps=10, dense_layers=()),
    "minimax_h3": dict(density=0.10, dense_steps=10, dense_layers=(0,)),
    "minimax_h3_rtx5090": dict(density=0.24, dense_steps=10, dense_layers=(0,)),
}

_FAMILIES = (("WanTransformer", "wan"), ("HunyuanVideoTransformer", "hunyuan_video"), ("MiniMaxH3", "minimax_h3"))


def model_family(pipe):
    """Family of a pipeline from its transformer's class name (reference models/__init__.py:13-21)."""
    name = type(pipe.transformer).__name__
    for prefix, family in _FAMILIES:
        if name.startswith(prefix):
            return family
    raise ValueError(f"unsupported transformer {name}")


def settings(family, preset=None, **overrides):
    """Attention settings of a family: its preset (or the named one of the same family) with `overrides` applied
    (reference models/__init__.py:24-31)."""
    preset = preset or family
    if preset not in PRESETS or not preset.startswith(family):
        have = sorted(p for p in PRESETS if p.startswith(family))
        raise ValueError(f"preset {preset!r} is not a {family} preset; have {have}")
    return {**PRESETS[preset], **overrides}


def enable(pipe, preset=None, gpu="auto", **overrides):
    """Route the pipeline's self-attention through EchoSparse attention and return the attention object
    (reference models/__init__.py:34-50). `overrides` replace preset values (density, dense_steps, dense_layers,
    refine_iters); `gpu` is "auto" or "mi355x"."""
    family = model_family(pipe)
    attention = EchoSparseAttention(**settings(family, preset, **overrides), gpu=gpu)
    if family == "wan":
        from . import wan as mod
    elif family == "hunyuan_video":
        from . import hunyuan_video as mod
    else:
        from . import minimax_h3 as mod
    mod.enable(pipe, attention)
    return attention
