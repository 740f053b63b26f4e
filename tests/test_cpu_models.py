"""Pipeline integrations on the CPU (reference echosparse/models/): the Morton order against a bit-by-bit
interleave, the clock against a scripted pipeline, presets, and each family's hooks on a small stand-in
transformer (diffusers is not installed: `fake_diffusers` provides the modules the integrations patch). The
attention object is a recording stand-in that computes dense attention, so the integration's token reordering,
routing and output assembly must reproduce the unpatched model exactly."""
import itertools

import numpy as np
import pytest
import torch

import fake_diffusers as fd
from fake_diffusers import sdpa


def brute_morton(t, y, x):
    code = 0
    for b in range(21):
        code |= ((x >> b) & 1) << (3 * b) | ((y >> b) & 1) << (3 * b + 1) | ((t >> b) & 1) << (3 * b + 2)
    return code


def test_morton_code_matches_bit_interleave():
    from self_trainable_or_free_attn_amd.models.common import morton_code
    rng = np.random.default_rng(0)
    pts = rng.integers(0, 1 << 21, size=(500, 3))
    pts = np.concatenate([pts, [[0, 0, 0], [0, 0, 1], [0, 1, 0], [1, 0, 0], [(1 << 21) - 1] * 3]])
    got = morton_code(*(torch.as_tensor(pts[:, i]) for i in range(3))).numpy()
    want = np.array([brute_morton(int(t), int(y), int(x)) for t, y, x in pts], dtype=np.int64)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("grid", [(2, 2, 2), (3, 5, 7), (21, 45, 80)])
def test_grid_morton_order(grid):
    from self_trainable_or_free_attn_amd.models.common import grid_morton_order
    perm, inv = grid_morton_order(*grid, torch.device("cpu"))
    n = grid[0] * grid[1] * grid[2]
    assert sorted(perm.tolist()) == list(range(n))
    assert torch.equal(perm[inv], torch.arange(n)) and torch.equal(inv[perm], torch.arange(n))
    # raster index r = (t * H + y) * W + x; the permuted list must have strictly increasing Morton codes
    t, rem = perm // (grid[1] * grid[2]), perm % (grid[1] * grid[2])
    y, x = rem // grid[2], rem % grid[2]
    codes = [brute_morton(int(a), int(b), int(c)) for a, b, c in zip(t, y, x)]
    assert all(c0 < c1 for c0, c1 in zip(codes, codes[1:]))
    if grid == (2, 2, 2):       # Morton and raster order coincide on a 2x2x2 cube
        assert torch.equal(perm, torch.arange(8))


def test_clock_follows_pipeline_calls():
    from self_trainable_or_free_attn_amd.models.common import Clock
    model = torch.nn.Linear(2, 2)
    pipe = fd.Pipe(model)
    resets = []
    clock = Clock(pipe, on_reset=[lambda: resets.append(1)])
    seen = []
    for video in range(2):
        pipe.scheduler.set_timesteps(3)
        assert len(resets) == video + 1 and (clock.step, clock.branch) == (0, -1)
        for step in range(3):
            for branch in range(2):
                model(torch.zeros(1, 2))
                for layer in range(3):
                    seen.append((clock.step, clock.branch, clock.layer))
                    clock.layer += 1
            pipe.scheduler.step()
    want = [(s, b, l) for s, b, l in itertools.product(range(3), range(2), range(3))]
    assert seen == want * 2
    assert pipe.scheduler.timesteps == [0, 1, 2]      # the wrapped methods still run


def test_presets_and_families():
    from self_trainable_or_free_attn_amd import models
    assert models.settings("wan") == dict(density=0.10, dense_steps=10, dense_layers=(0,))
    assert models.settings("hunyuan_video", density=0.2)["density"] == 0.2
    assert models.settings("minimax_h3", "minimax_h3_rtx5090")["density"] == 0.24
    with pytest.raises(ValueError, match="is not a wan preset"):
        models.settings("wan", "hunyuan_video")
    mods = fd.install()
    assert models.model_family(fd.Pipe(fd.WanTransformer3DModel(mods["transformer_wan"]))) == "wan"
    with pytest.raises(ValueError, match="unsupported transformer"):
        models.model_family(fd.Pipe(torch.nn.Linear(1, 1)))


class RecordingAttention:
    """Stands in for EchoSparseAttention: dense attention in float32, records every call's arguments."""

    def __init__(self):
        self.calls, self.resets = [], 0

    def reset(self):
        self.resets += 1

    def __call__(self, q, k, v, step, branch, layer, sink=None, rows=None):
        self.calls.append(dict(step=step, branch=branch, layer=layer, sink=sink, rows=rows, L=q.shape[1]))
        return sdpa(q, k, v)


def _dense_model_output(model, mod, *args, **kwargs):
    saved = mod.dispatch_attention_fn
    mod.dispatch_attention_fn = fd.default_dispatch
    try:
        with torch.no_grad():
            return model(*args, **kwargs)
    finally:
        mod.dispatch_attention_fn = saved


def test_wan_hooks_reorder_and_route(monkeypatch):
    mods = fd.install()
    tw = mods["transformer_wan"]
    torch.manual_seed(0)
    model = fd.WanTransformer3DModel(tw, depth=3)
    lat, enc = torch.randn(1, 4, 3, 12, 10), torch.randn(1, 9, 64)
    want = _dense_model_output(model, tw, lat, enc)
    from self_trainable_or_free_attn_amd.models import wan
    monkeypatch.setattr(wan, "dense_attention", lambda q, k, v: sdpa(q, k, v))
    monkeypatch.setattr(tw, "dispatch_attention_fn", tw.dispatch_attention_fn)
    pipe = fd.Pipe(model)
    att = RecordingAttention()
    wan.enable(pipe, att)
    assert tw.dispatch_attention_fn is wan._dispatch
    pipe.scheduler.set_timesteps(2)
    with torch.no_grad():
        for step in range(2):
            for _branch in range(2):
                got = model(lat, enc)
                torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
            pipe.scheduler.step()
    assert att.resets == 1
    assert [(c["step"], c["branch"], c["layer"]) for c in att.calls] == \
        [(s, b, l) for s in range(2) for b in range(2) for l in range(3)]
    assert all(c["L"] == 3 * 6 * 5 and c["sink"] is None for c in att.calls)


def test_hunyuan_hooks_crop_sink_and_text_rows(monkeypatch):
    mods = fd.install()
    hv = mods["transformer_hunyuan_video"]
    torch.manual_seed(1)
    model = fd.HunyuanVideoTransformer3DModel(hv)
    lat, txt = torch.randn(1, 4, 2, 16, 18), torch.randn(1, 11, 64)
    tmask = torch.zeros(1, 11, dtype=torch.bool)
    tmask[:, :6] = True
    vl = 2 * 8 * 9
    before = fd.default_dispatch.calls
    want = _dense_model_output(model, hv, lat, txt, tmask)
    from self_trainable_or_free_attn_amd.models import hunyuan_video
    monkeypatch.setattr(hunyuan_video, "dense_attention", lambda q, k, v: sdpa(q, k, v))
    monkeypatch.setattr(hv, "dispatch_attention_fn", hv.dispatch_attention_fn)
    monkeypatch.setattr(hunyuan_video, "_original_dispatch", fd.default_dispatch)
    pipe = fd.Pipe(model)
    att = RecordingAttention()
    hunyuan_video.enable(pipe, att)
    pipe.scheduler.set_timesteps(1)
    with torch.no_grad():
        got = model(lat, txt, tmask)
    # padded text rows: the integration writes zeros there, the masked dense model does not; compare valid rows
    L = vl + 6
    torch.testing.assert_close(got[:, :L], want[:, :L], rtol=1e-5, atol=1e-5)
    assert fd.default_dispatch.calls - before == 3 + 1      # 3 dense-model calls, then the refiner call
    assert [c["sink"] for c in att.calls] == [vl // 64] * 2 and [c["L"] for c in att.calls] == [L] * 2
    assert [c["layer"] for c in att.calls] == [0, 1]


def test_minimax_hooks_packed_sequence(monkeypatch):
    mods = fd.install()
    th3 = mods["transformer_minimax_h3"]
    torch.manual_seed(2)
    model = fd.MiniMaxH3Transformer(th3)
    prefix, grid = 23, (3, 6, 7)
    pos, vi = fd.h3_positions(prefix, *grid)
    L = prefix + grid[0] * grid[1] * grid[2]
    x = torch.randn(1, L, 64)
    want = _dense_model_output(model, th3, x, position_ids=pos, video_indices=vi)
    from self_trainable_or_free_attn_amd.models import minimax_h3
    monkeypatch.setattr(minimax_h3, "dense_attention", lambda q, k, v: sdpa(q, k, v))
    monkeypatch.setattr(th3, "dispatch_attention_fn", th3.dispatch_attention_fn)
    monkeypatch.setattr(minimax_h3, "_original_dispatch", fd.default_dispatch)
    pipe = fd.Pipe(model)
    att = RecordingAttention()
    impl = minimax_h3.enable(pipe, att)
    pipe.scheduler.set_timesteps(1)
    with torch.no_grad():
        got = model(x, position_ids=pos, video_indices=vi)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    nv = L - prefix
    assert impl.layout.video_start == prefix and impl.layout.video == nv
    assert [(c["sink"], c["rows"], c["L"]) for c in att.calls] == [(nv // 64, nv, L)] * 2
    # the video part of the packed order is the Morton order of the ranked rotary coordinates
    from self_trainable_or_free_attn_amd.models.common import grid_morton_order
    perm, _ = grid_morton_order(*grid, torch.device("cpu"))
    assert torch.equal(impl.layout.packed_to_original[:nv], perm + prefix)
    assert torch.equal(impl.layout.packed_to_original[nv:], torch.arange(prefix))
