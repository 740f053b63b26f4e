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
    from self_trainable_or_free_attn_amd.models import common, wan
    monkeypatch.setattr(common, "dense_attention", lambda q, k, v: sdpa(q, k, v))
    monkeypatch.setattr(tw, "dispatch_attention_fn", tw.dispatch_attention_fn)
    pipe = fd.Pipe(model)
    att = RecordingAttention()
    wan.install(pipe, att)
    assert tw.dispatch_attention_fn.original is fd.default_dispatch
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
    from self_trainable_or_free_attn_amd.models import common, hunyuan_video
    monkeypatch.setattr(common, "dense_attention", lambda q, k, v: sdpa(q, k, v))
    monkeypatch.setattr(hv, "dispatch_attention_fn", fd.default_dispatch)
    pipe = fd.Pipe(model)
    att = RecordingAttention()
    hunyuan_video.install(pipe, att)
    pipe.scheduler.set_timesteps(1)
    with torch.no_grad():
        got = model(lat, txt, tmask)
    # padded text rows: the integration writes zeros there, the masked dense model does not; compare valid rows
    L = vl + 6
    torch.testing.assert_close(got[:, :L], want[:, :L], rtol=1e-5, atol=1e-5)
    assert fd.default_dispatch.calls - before == 3 + 1      # 3 dense-model calls, then the refiner call
    # only the video rows enter the sparse kernels; the text rows are computed densely
    assert [(c["sink"], c["rows"], c["L"]) for c in att.calls] == [(vl // 64, vl, L)] * 2
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
    from self_trainable_or_free_attn_amd.models import common, minimax_h3
    monkeypatch.setattr(common, "dense_attention", lambda q, k, v: sdpa(q, k, v))
    monkeypatch.setattr(th3, "dispatch_attention_fn", fd.default_dispatch)
    pipe = fd.Pipe(model)
    att = RecordingAttention()
    impl = minimax_h3.install(pipe, att)
    pipe.scheduler.set_timesteps(1)
    with torch.no_grad():
        got = model(x, position_ids=pos, video_indices=vi)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    nv = L - prefix
    assert impl.layout.start == prefix and impl.layout.n == nv
    assert [(c["sink"], c["rows"], c["L"]) for c in att.calls] == [(nv // 64, nv, L)] * 2
    # the video part of the packed order is the Morton order of the ranked rotary coordinates
    from self_trainable_or_free_attn_amd.models.common import grid_morton_order
    perm, _ = grid_morton_order(*grid, torch.device("cpu"))
    assert torch.equal(impl.layout.gather[:nv], perm + prefix)
    assert torch.equal(impl.layout.gather[nv:], torch.arange(prefix))


def test_morton_known_answer():
    """Reference tests/test_attention.py:152-155: the first tokens of a 5 x 6 x 7 grid in Morton order."""
    from self_trainable_or_free_attn_amd.models.common import grid_morton_order
    perm, inv = grid_morton_order(5, 6, 7, torch.device("cpu"))
    assert torch.equal(perm[inv], torch.arange(5 * 6 * 7))
    assert perm[:8].tolist() == [0, 1, 7, 8, 42, 43, 49, 50]


def test_h3_layout_strided_time_axis():
    """Reference tests/test_api.py:146-166 (the layout part): a prefix of text, conditioning-video and audio tokens,
    then a 2 x 3 x 4 target video whose rotary t coordinate steps by 2; the packed order is the video in the Morton
    order of the ranked coordinates, then the prefix in its own order."""
    fd.install()
    from self_trainable_or_free_attn_amd.models.common import morton_order
    from self_trainable_or_free_attn_amd.models.minimax_h3 import packed_layout
    t, y, x = torch.meshgrid(torch.arange(0, 4, 2), torch.arange(3), torch.arange(4), indexing="ij")
    video = torch.stack([t.flatten(), y.flatten(), x.flatten()], 1)
    pos = torch.cat([torch.zeros(9, 3, dtype=torch.long), video])
    L, vs = pos.shape[0], 9
    layout = packed_layout(pos, torch.cat([torch.arange(3, 7), torch.arange(vs, L)]))
    perm, _ = morton_order(video[:, 0] // 2, video[:, 1], video[:, 2])
    assert layout.n == L - vs and layout.start == vs
    assert torch.equal(layout.gather[:L - vs], perm + vs)
    assert torch.equal(layout.gather[L - vs:], torch.arange(vs))
    assert torch.equal(torch.sort(layout.gather).values, torch.arange(L))


def test_enable_and_attention_agree(monkeypatch):
    """Reference tests/test_api.py:86-99: the package-level enable builds the attention from the named preset and
    hands that same object to the family's hooks."""
    import sys
    import types
    import self_trainable_or_free_attn_amd as pkg
    from self_trainable_or_free_attn_amd import models
    seen = {}
    fake = types.ModuleType("self_trainable_or_free_attn_amd.models.minimax_h3")
    fake.TRANSFORMER_PREFIX = "MiniMaxH3"
    fake.install = lambda pipe, attention: seen.update(attention=attention)
    monkeypatch.setitem(sys.modules, fake.__name__, fake)
    monkeypatch.setattr(models, "minimax_h3", fake, raising=False)
    pipe = types.SimpleNamespace(transformer=type("MiniMaxH3Transformer", (), {})())
    attn = pkg.enable(pipe, preset="minimax_h3_rtx5090", gpu="mi355x", refine_iters=6)
    assert seen["attention"] is attn
    assert (attn.density, attn.dense_steps, attn.dense_layers, attn.gpu) == (0.24, 10, {0}, "mi355x")
    with pytest.raises(ValueError, match="gpu must be"):
        pkg.enable(pipe, gpu="sm120")


def test_device_change_releases_old_history(monkeypatch):
    """Reference tests/test_api.py:64-83: state and scratch survive calls on one device and are dropped when the
    inputs move to another."""
    import types
    from self_trainable_or_free_attn_amd import EchoSparseAttention, attention, backends
    monkeypatch.setattr(backends, "resolve", lambda gpu, device: "mi355x")
    monkeypatch.setattr(backends, "kernels", lambda name: None)
    monkeypatch.setattr(attention, "dense_attention", lambda q, k, v: q)
    attn = EchoSparseAttention()
    q = types.SimpleNamespace(shape=(1, 128, 1, 128), device=torch.device("cuda:0"))
    attn(q, q, q, step=0, branch=0, layer=0)
    previous = object()
    attn._states[1] = previous
    attn._buffers = attn._plan_scratch = previous
    attn(q, q, q, step=0, branch=0, layer=0)
    assert attn._states[1] is previous and attn._buffers is previous
    q.device = torch.device("cuda:1")
    attn(q, q, q, step=0, branch=0, layer=0)
    assert not attn._states
    assert attn._buffers is None and attn._plan_scratch is None


def test_target_video_start_is_the_last_consecutive_run():
    """The split of H3's video_indices against a brute-force walk back from the end, on random ascending index
    lists made of several runs."""
    fd.install()
    from self_trainable_or_free_attn_amd.models.minimax_h3 import target_video_start
    g = np.random.default_rng(7)
    for _ in range(200):
        runs, pos, idx = g.integers(1, 5), 0, []
        for _r in range(runs):
            pos += int(g.integers(1, 6))
            n = int(g.integers(1, 9))
            idx.extend(range(pos, pos + n))
            pos += n
        i = len(idx) - 1
        while i > 0 and idx[i - 1] == idx[i] - 1:
            i -= 1
        assert target_video_start(torch.tensor(idx)) == i


def test_sink_layout_rows_and_padding():
    """A joint sequence with a prefix, a video span, a suffix and padding: video rows come from the sparse call in
    the original order, other valid rows from dense attention over every valid key, padding rows are zero, and the
    sparse call sees the video first with sink = n // 64 and rows = n."""
    from self_trainable_or_free_attn_amd.models import common
    torch.manual_seed(3)
    start, n, valid, total = 5, 150, 170, 180
    perm = torch.randperm(n)
    lay = common.SinkLayout(start, perm, valid)
    q, k, v = (torch.randn(1, total, 2, 16) for _ in range(3))
    seen = {}

    def attention(qp, kp, vp, step, branch, layer, sink=None, rows=None):
        seen.update(sink=sink, rows=rows, q=qp)
        return sdpa(qp, kp, vp)

    clock = type("C", (), dict(step=0, branch=0, layer=4))()
    dense = common.dense_attention
    common.dense_attention = lambda a, b, c: sdpa(a, b, c)
    try:
        out = lay(attention, clock, q, k, v)
    finally:
        common.dense_attention = dense
    assert (seen["sink"], seen["rows"], clock.layer) == (n // 64, n, 5)
    assert torch.equal(seen["q"][:, :n], q[:, start + perm])
    want = sdpa(q[:, :valid], k[:, :valid], v[:, :valid])
    torch.testing.assert_close(out[:, :valid], want, rtol=1e-5, atol=1e-5)
    assert (out[:, valid:] == 0).all()
    with pytest.raises(ValueError, match="outside"):
        common.SinkLayout(30, perm, valid)


def test_model_family_accepts_subclasses():
    from self_trainable_or_free_attn_amd import models
    mods = fd.install()

    class MyWan(fd.WanTransformer3DModel):
        pass

    assert models.model_family(fd.Pipe(MyWan(mods["transformer_wan"]))) == "wan"
    assert models.family_presets("minimax_h3") == ["minimax_h3", "minimax_h3_rtx5090"]
