"""Pipeline integrations (behaviour of the reference's echosparse/models/__init__.py): `enable(pipe)` routes a
diffusers video pipeline's self-attention through EchoSparseAttention on MI355X.

    wan              diffusers WanPipeline (Wan2.1): self-attention sparse, cross-attention dense
    hunyuan_video    diffusers HunyuanVideoPipeline: video rows sparse with the text tokens as a sink
    minimax_h3       the minimax-h3 branch of diffusers: target-video rows sparse, the prefix as a sink

Each family module names the transformer class it handles (`TRANSFORMER_PREFIX`) and installs its routes with
`install(pipe, attention)`; diffusers is imported only inside `install`, so the package imports without it.
"""
import importlib

from ..attention import EchoSparseAttention

# The settings of the reference's reported results (reference models/__init__.py:5-10), kept as published: a
# family's own preset carries its name, variants append a suffix.
PRESETS = {
    "wan": dict(density=0.10, dense_steps=10, dense_layers=(0,)),
    "hunyuan_video": dict(density=0.10, dense_steps=10, dense_layers=()),
    "minimax_h3": dict(density=0.10, dense_steps=10, dense_layers=(0,)),
    "minimax_h3_rtx5090": dict(density=0.24, dense_steps=10, dense_layers=(0,)),
}

FAMILIES = ("wan", "hunyuan_video", "minimax_h3")


def _module(family):
    return importlib.import_module(f".{family}", __name__)


def model_family(pipe):
    """Family of a pipeline: the first family whose transformer prefix starts the name of the transformer's class
    or of one of its base classes (subclasses of a supported transformer are supported)."""
    classes = [c.__name__ for c in type(pipe.transformer).__mro__]
    for family in FAMILIES:
        prefix = _module(family).TRANSFORMER_PREFIX
        if any(name.startswith(prefix) for name in classes):
            return family
    raise ValueError(f"unsupported transformer {classes[0]}")


def family_presets(family):
    """Names of the presets of a family: its own and its suffixed variants."""
    return sorted(name for name in PRESETS if name == family or name.startswith(family + "_"))


def settings(family, preset=None, **overrides):
    """Attention settings of a family: its preset (or the named variant) with `overrides` applied (reference
    models/__init__.py:24-31)."""
    name = family if preset is None else preset
    allowed = family_presets(family)
    if name not in allowed:
        raise ValueError(f"preset {name!r} is not a {family} preset; have {allowed}")
    merged = dict(PRESETS[name])
    merged.update(overrides)
    return merged


def enable(pipe, preset=None, gpu="auto", **overrides):
    """Route the pipeline's self-attention through EchoSparse attention and return the attention object
    (reference models/__init__.py:34-50). `overrides` replace preset values (density, dense_steps, dense_layers,
    refine_iters); `gpu` is "auto" or "mi355x"."""
    family = model_family(pipe)
    attention = EchoSparseAttention(gpu=gpu, **settings(family, preset, **overrides))
    _module(family).install(pipe, attention)
    return attention
