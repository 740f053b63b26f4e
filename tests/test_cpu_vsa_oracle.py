"""Pins of the VSA oracle (oracle/vsa_ref.py) and of the host-side VSA modules (layout, dispatch, operator
argument checks), CPU only. Each check is independent of the formula it pins: known answers from the reference's
own tests, library routines (torch scaled_dot_product_attention, torch.autograd, Python's stable sort), brute force
on tiny inputs, and invariants."""
import math

import numpy as np
import pytest
import torch

from oracle import vsa_ref as ref
from oracle.bf16 import round_bf16


# --------------------------------------------------------------------------- pooling
def test_pool_matches_float64_means_and_skips_padding():
    g = np.random.default_rng(0)
    cnt = [64, 10, 1, 33]
    x = g.standard_normal((1, 2, 256, 8)).astype(np.float32)
    for b, c in enumerate(cnt):
        x[:, :, b * 64 + c:(b + 1) * 64] = np.nan  # padding is never read
    for R in (4, 8, 16, 32):
        grp, blk = ref.pool(x, cnt, R)
        assert np.isfinite(grp).all() and np.isfinite(blk).all()
        G = 64 // R
        for b, c in enumerate(cnt):
            want = x[:, :, b * 64:b * 64 + c].astype(np.float64).mean(2)
            assert np.abs(blk[:, :, b] - want).max() <= 2.0 ** -7 * np.abs(want).max() + 1e-6
            for gi in range(G):
                r0, r1 = gi * R, min(gi * R + R, c)
                if r1 <= r0:
                    assert (grp[:, :, b * G + gi] == 0).all()
                else:
                    w = x[:, :, b * 64 + r0:b * 64 + r1].astype(np.float64).mean(2)
                    assert np.abs(grp[:, :, b * G + gi] - w).max() <= 2.0 ** -7 * np.abs(w).max() + 1e-6


def test_bf16_rounding_matches_torch():
    x = np.random.default_rng(1).standard_normal(10000).astype(np.float32) * 100
    assert np.array_equal(round_bf16(x), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_f16_rounding_matches_torch():
    from oracle.bf16 import round_f16
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(10000) * 100, rng.standard_normal(1000) * 1e5,
                        rng.standard_normal(1000) * 1e-6]).astype(np.float32)
    assert np.array_equal(round_f16(x), torch.from_numpy(x).to(torch.float16).float().numpy())


# --------------------------------------------------------------------------- selections
def test_row_topk_known_answers():
    """reference tests/test_vsa.py:67-73"""
    s = np.array([[[0.5, 0.0, -0.0, 0.5, 0.25, 0.0]]])
    assert ref.row_topk_mask(s, 3).tolist() == [[[True, False, False, True, True, False]]]
    assert ref.row_topk_mask(s, 4).tolist() == [[[True, True, False, True, True, False]]]
    assert ref.row_topk_mask(s, 5).tolist() == [[[True, True, True, True, True, False]]]
    assert ref.row_topk_mask(s, 6).all() and not ref.row_topk_mask(s, 0).any()
    assert ref.row_topk_mask(s, 99).all()


def test_row_topk_brute_force():
    g = np.random.default_rng(2)
    s = g.integers(-3, 4, (4, 30)).astype(np.float64) / 2
    for K in (0, 1, 5, 29, 30):
        m = ref.row_topk_mask(s, K)
        for r in range(4):
            order = sorted(range(30), key=lambda j: (-s[r, j], j))[:K]
            assert sorted(np.nonzero(m[r])[0].tolist()) == sorted(order)


def test_global_topk_brute_force_and_count():
    g = np.random.default_rng(3)
    s = g.integers(-4, 5, (1, 2, 7, 7)).astype(np.float64)
    s[0, 0, 3] = -0.0
    for budget in (0, 1, 10, 48, 49, 1000):
        m = ref.global_topk_mask(s, budget)
        assert (m.reshape(2, -1).sum(1) == min(budget, 49)).all()
        for h in range(2):
            flat = s[0, h].reshape(-1) + 0.0
            want = sorted(range(49), key=lambda j: (-flat[j], j))[:budget]
            assert sorted(np.nonzero(m[0, h].reshape(-1))[0].tolist()) == sorted(want)


def test_csr_round_trip():
    m = np.random.default_rng(4).random((2, 3, 9, 9)) < 0.3
    ptr, idx = ref.csr_from_mask(m)
    assert np.array_equal(ref.mask_from_csr(ptr, idx, 9), m)
    assert ptr[0, 0, 0] == 0 and ptr[-1, -1, -1] == idx.size


# --------------------------------------------------------------------------- PSP router
def test_psp_rows_sum_to_one_and_norms():
    g = np.random.default_rng(5)
    R, cnt = 16, [64] * 5
    qr = g.standard_normal((1, 2, 20, 16))
    kr = g.standard_normal((1, 2, 20, 16))
    s0 = ref.psp_scores(qr, kr, cnt, R, 0)
    s1 = ref.psp_scores(qr, kr, cnt, R, 1)
    assert np.allclose(s0.sum(-1), 1.0)
    assert np.allclose(s1, s0 / 4)


def test_psp_brute_force_tiny():
    g = np.random.default_rng(6)
    R, cnt = 32, [64, 20]            # G = 2; block 1's second group is empty
    qr = g.standard_normal((1, 1, 4, 4))
    kr = g.standard_normal((1, 1, 4, 4))
    got = ref.psp_scores(qr, kr, cnt, R, 0)
    valid = [True, True, True, False]
    want = np.zeros((2, 2))
    for a in range(4):
        if not valid[a]:
            continue
        logits = [qr[0, 0, a] @ kr[0, 0, c] / 2.0 if valid[c] else -np.inf for c in range(4)]
        mx = max(logits)
        e = [math.exp(t - mx) if np.isfinite(t) else 0.0 for t in logits]
        for c in range(4):
            want[a // 2, c // 2] += e[c] / sum(e)
    want[0] /= 2
    want[1] /= 1
    assert np.allclose(got[0, 0], want)


# --------------------------------------------------------------------------- fine attention
def _inputs(seed, cnt, D=16, H=2):
    g = torch.Generator().manual_seed(seed)
    L = len(cnt) * 64
    valid = torch.as_tensor(ref.token_valid(cnt, L))[None, None, :, None].double()
    return [(torch.randn(1, H, L, D, generator=g, dtype=torch.float64) * valid) for _ in range(3)]


def test_fine_full_mask_is_dense_attention():
    cnt = [64, 64, 64]
    q, k, v = _inputs(0, cnt)
    o, lse = ref.fine_attention(q.numpy(), k.numpy(), v.numpy(), cnt, np.ones((1, 2, 3, 3), bool))
    want = torch.nn.functional.scaled_dot_product_attention(q, k, v)
    assert np.allclose(o, want.numpy(), atol=1e-12)
    s = (q @ k.transpose(-1, -2)) / math.sqrt(16)
    assert np.allclose(lse, torch.logsumexp(s, -1).numpy())


def test_fine_empty_rows_padding_and_block_order():
    cnt = [64, 30, 64, 5]
    q, k, v = _inputs(1, cnt)
    m = np.random.default_rng(7).random((1, 2, 4, 4)) < 0.5
    m[:, :, 2] = False
    o, lse = ref.fine_attention(q.numpy(), k.numpy(), v.numpy(), cnt, m)
    assert (o[:, :, 128:192] == 0).all() and np.isneginf(lse[:, :, 128:192]).all()
    pad = ~ref.token_valid(cnt, 256)
    assert (o[:, :, pad] == 0).all() and np.isneginf(lse[:, :, pad]).all()
    # swapping two kv blocks (keys, values, mask columns together) leaves O unchanged
    perm = np.array([0, 2, 1, 3])
    tok = np.concatenate([np.arange(64) + 64 * b for b in perm])
    cnt_p = [cnt[b] for b in perm]
    k2, v2 = k.numpy()[:, :, tok], v.numpy()[:, :, tok]
    # query positions keep their blocks; only key-side columns move, so recompute with permuted keys by hand
    valid_k = ref.token_valid(cnt, 256)[tok]
    blk_q = np.arange(256) // 64
    allowed = m[:, :, blk_q][:, :, :, perm[np.arange(256) // 64]] & valid_k[None, None, None, :]
    s = np.einsum("bhid,bhjd->bhij", q.numpy(), k2) / 4.0
    s = np.where(allowed, s, -np.inf)
    has = allowed.any(-1) & ref.token_valid(cnt, 256)[None, None, :]
    mx = np.where(has, s.max(-1), 0)
    p = np.where(allowed, np.exp(s - mx[..., None]), 0)
    o2 = np.einsum("bhij,bhjd->bhid", p / np.where(has, p.sum(-1), 1)[..., None], v2) * has[..., None]
    assert np.allclose(o, o2)
    assert cnt_p == [64, 64, 30, 5]


def test_fine_backward_matches_autograd():
    cnt = [64, 40, 64]
    q, k, v = _inputs(2, cnt)
    m = np.random.default_rng(8).random((1, 2, 3, 3)) < 0.6
    m[:, :, 1] = False
    dout = torch.randn(q.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(9))
    dout = dout * torch.as_tensor(ref.token_valid(cnt, 192))[None, None, :, None]
    got = ref.fine_backward(q.numpy(), k.numpy(), v.numpy(), cnt, m, dout.numpy())
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v)]
    o = ref.vsa_output(*leaves, None, cnt, m, pooled=None) - ref.vsa_output(*[x.detach() for x in leaves], None, cnt,
                                                                               np.zeros_like(m), pooled=None)
    # vsa_output includes the coarse branch; fine-only autograd via a torch restatement below
    blk = torch.arange(192) // 64
    valid = torch.as_tensor(ref.token_valid(cnt, 192))
    allowed = torch.as_tensor(m)[:, :, blk][:, :, :, blk] & valid[None, None, None, :]
    s = (leaves[0] @ leaves[1].transpose(-1, -2)) / 4.0
    s = s.masked_fill(~allowed, float("-inf"))
    has = allowed.any(-1, keepdim=True) & valid[None, None, :, None]
    p = torch.softmax(torch.where(has, s, torch.zeros_like(s)), -1) * has
    want = torch.autograd.grad(p @ leaves[2], leaves, dout)
    for a, b in zip(got, want):
        assert np.allclose(a, b.numpy(), atol=1e-10)
    assert o.shape == q.shape


def test_empty_mask_leaves_only_coarse_branch():
    """reference tests/test_vsa.py:76-84: Q = K = V = 1, no kv block -> O = O_c = 1."""
    q, k, v = (torch.ones(1, 1, 64, 16, dtype=torch.float64, requires_grad=True) for _ in range(3))
    o = ref.vsa_output(q, k, v, None, [64], np.zeros((1, 1, 1, 1), bool))
    assert torch.allclose(o, torch.ones_like(o))
    for gr in torch.autograd.grad(o.sum(), (q, k, v)):
        assert torch.isfinite(gr).all()


# --------------------------------------------------------------------------- split plan and merges
def test_plan_reference_hand_case_and_cover():
    # one head, 4 rows with lengths 5, 1, 9, 0; chunk 2 -> thr = 3: rows 0 and 2 split into 3 and 5 chunks
    ptr = np.array([[[0, 5, 6, 15, 15]]])
    tasks, merges, info = ref.plan_reference(ptr, 2, 100)
    assert merges == [[0, 0, 3, 0], [2, 3, 5, 0]]
    assert info == [3 + 5 + 2, 2, 8, 4, 2, 1, 3, 15]
    assert tasks[:3] == [[0, 0, 1, 0], [0, 1, 3, 1], [0, 3, 5, 2]]
    assert tasks[-2:] == [[1, 5, 6, -1], [3, 15, 15, -1]]
    cover = np.zeros(15, int)
    for _, b, e, _ in tasks:
        cover[b:e] += 1
    assert (cover == 1).all()
    # slot cap: row 2 does not fit in 4 slots and runs direct, as does everything after it
    _, merges, info = ref.plan_reference(ptr, 2, 4)
    assert merges == [[0, 0, 3, 0]] and info[2] == 3
    # budget below the eligible count: nothing splits
    _, merges, info = ref.plan_reference(ptr, 2, 100, budget=1)
    assert merges == [] and info[5] == 0


def test_merge_fwd_equals_unsplit_softmax():
    g = np.random.default_rng(10)
    s = g.standard_normal(40)
    v = g.standard_normal((40, 3))
    parts = [(0, 13), (13, 30), (30, 40)]
    po, pl = [], []
    for a, b in parts:
        e = np.exp(s[a:b])
        po.append(e @ v[a:b] / e.sum())
        pl.append(np.log2(e.sum()))
    o, lse = ref.merge_fwd(np.array(po)[:, None], np.array(pl)[:, None])
    e = np.exp(s)
    assert np.allclose(o[0], e @ v / e.sum()) and np.isclose(lse[0], np.log(e.sum()))


# --------------------------------------------------------------------------- host modules
def test_layout_round_trip_and_reference_order():
    from self_trainable_or_free_attn_amd.vsa import layout
    for lay in (layout.build_layout((6, 9, 10), R=16), layout.sequence_layout(300),
                layout.build_layout((5, 4, 8), tile=(1, 8, 8), sub=(1, 2, 2))):
        n = lay.scatter.numel()
        assert int(lay.blk_cnt.sum()) == n and lay.padded_len == lay.num_blocks * 64
        x = torch.randn(1, 2, n, 8, dtype=torch.float64, requires_grad=True)
        xb = layout.to_blocked(x, lay)
        assert (xb[:, :, lay.gather < 0] == 0).all()
        assert torch.equal(layout.from_blocked(xb, lay), x)
        assert torch.equal(torch.as_tensor(ref.token_valid(lay.blk_cnt.numpy(), lay.padded_len)), lay.gather >= 0)
    # brute-force order of a boundary-cut grid: tiles in raster order, sub-cube major inside, existing tokens first
    T, Hh, W, tile, sub = 5, 6, 7, (4, 4, 4), (1, 4, 4)
    lay = layout.build_layout((T, Hh, W), tile=tile, sub=sub)
    want = []
    for t0 in range(0, T, 4):
        for h0 in range(0, Hh, 4):
            for w0 in range(0, W, 4):
                blk = []
                for a in range(4):
                    for b in range(1):
                        for c in range(1):
                            for x in range(1):
                                for y in range(4):
                                    for z in range(4):
                                        t, h, w = t0 + a + x, h0 + b * 4 + y, w0 + c * 4 + z
                                        if t < T and h < Hh and w < W:
                                            blk.append((t * Hh + h) * W + w)
                want += blk + [-1] * (64 - len(blk))
    assert lay.gather.tolist() == want


def test_bwd_variant_precedence():
    from self_trainable_or_free_attn_amd.vsa.dispatch import select_bwd_variant
    assert select_bwd_variant(1, 2, 64, 128, -1) == (2, "auto")
    assert select_bwd_variant(1, 2, 64, 128, -1, call=0) == (0, "call")
    assert select_bwd_variant(1, 2, 64, 128, -1, override=1) == (1, "set_bwd_variant")
    assert select_bwd_variant(1, 2, 64, 128, -1, environ={"ECHOSPARSE_VSA_BWD_VARIANT": "0"}) == (0, "environment")
    with pytest.raises(ValueError):
        select_bwd_variant(1, 2, 64, 128, -1, call=3)
    with pytest.raises(ValueError):
        select_bwd_variant(1, 2, 64, 128, -1, environ={"ECHOSPARSE_VSA_BWD_VARIANT": "x"})


def test_split_dataclasses_validate():
    from self_trainable_or_free_attn_amd.vsa import SplitKV, SplitPolicy
    with pytest.raises(ValueError):
        SplitKV(chunk=0)
    with pytest.raises(TypeError):
        SplitKV(policy="auto")
    with pytest.raises(TypeError):
        SplitPolicy(min_chunks=True)
    with pytest.raises(ValueError):
        SplitPolicy(rel_mean=float("inf"))
    assert SplitKV.auto().policy == SplitPolicy()
    from self_trainable_or_free_attn_amd.vsa.ops import split_slots
    assert split_slots(1000, 64, 100, 10 ** 9) == 2 * 16 and split_slots(1000, 64, 100, 250) == 2


def test_import_does_not_load_the_library():
    import subprocess
    import sys
    code = ("import sys, self_trainable_or_free_attn_amd.vsa; "
            "assert self_trainable_or_free_attn_amd._lib._lib is None")
    subprocess.run([sys.executable, "-c", code], check=True, cwd=__file__.rsplit("/tests/", 1)[0])


# --------------------------------------------------------------------------- three-tier representatives
def _rep_inputs(seed, cnt, D=16):
    g = torch.Generator().manual_seed(seed)
    L = len(cnt) * 64
    valid = torch.as_tensor(ref.token_valid(cnt, L))[None, None, :, None].double()
    return [(torch.randn(1, 2, L, D, generator=g, dtype=torch.float64) * valid) for _ in range(3)]


def test_rep_tier_a_only_is_fine_attention():
    cnt = [64, 40, 64, 9]
    q, k, v = _rep_inputs(0, cnt)
    m = np.random.default_rng(1).random((1, 2, 4, 4)) < 0.5
    o, lse = ref.rep_fine_torch(q, k, v, cnt, m, m | (np.random.default_rng(2).random((1, 2, 4, 4)) < 0.5), 4, 1)
    wo, wl = ref.fine_attention(q.numpy(), k.numpy(), v.numpy(), cnt, m)
    assert np.allclose(o.numpy(), wo) and np.allclose(np.where(np.isfinite(wl), lse.numpy(), 0), np.where(np.isfinite(wl), wl, 0))


def test_rep_constant_groups_equal_dense_attention():
    """A representative of c identical tokens with + ln c is exactly those c columns: with every group constant,
    any tier assignment gives dense attention over the valid tokens."""
    cnt = [64, 64, 37]
    D, RM = 8, 4
    g = torch.Generator().manual_seed(3)
    L = 192
    base = torch.randn(1, 1, L // 16, D, generator=g, dtype=torch.float64)
    k = base.repeat_interleave(16, 2)          # constant over every 16-token group
    v = torch.randn(1, 1, L // 16, D, generator=g, dtype=torch.float64).repeat_interleave(16, 2)
    q = torch.randn(1, 1, L, D, generator=g, dtype=torch.float64)
    valid = torch.as_tensor(ref.token_valid(cnt, L))[None, None, :, None].double()
    q, k, v = q * valid, k * valid, v * valid
    ma = np.array([[[[1, 0, 0], [0, 0, 1], [0, 0, 0]]]], bool)
    mab = np.ones_like(ma)  # tiers A and B only: the groups are constant, the blocks are not
    o, _ = ref.rep_fine_torch(q, k, v, cnt, ma, mab, RM)
    wo, _ = ref.fine_attention(q.numpy(), k.numpy(), v.numpy(), cnt, np.ones((1, 1, 3, 3), bool))
    assert np.allclose(o.numpy(), wo, atol=1e-12)
    # the tail tier alone with blocks made constant
    kc = k.reshape(1, 1, 3, 64, D)[:, :, :, :1].expand(1, 1, 3, 64, D).reshape(1, 1, L, D) * valid
    vc = v.reshape(1, 1, 3, 64, D)[:, :, :, :1].expand(1, 1, 3, 64, D).reshape(1, 1, L, D) * valid
    o, _ = ref.rep_fine_torch(q, kc, vc, cnt, np.zeros_like(ma), np.zeros_like(ma), RM)
    wo, _ = ref.fine_attention(q.numpy(), kc.numpy(), vc.numpy(), cnt, np.ones((1, 1, 3, 3), bool))
    assert np.allclose(o.numpy(), wo, atol=1e-12)


@pytest.mark.parametrize("kmeans", [False, True])
def test_rep_fine_head_equals_the_autograd_graph(kmeans):
    """The blockwise analytic three-tier forward / backward of one head equals rep_fine_torch and its autograd
    gradients: partial blocks (one with a single token, so groups are empty), a row with no tier-A block, a row
    with no tier-C block, contiguous and k-means groups, a given stored O for delta."""
    cnt = [64, 64, 37, 64, 1, 64, 20, 50]
    NB, RM, D = len(cnt), 4, 16
    L = NB * 64
    g = torch.Generator().manual_seed(7)
    valid = torch.as_tensor(ref.token_valid(cnt, L))[None, None, :, None].double()
    q, k, v, do = (torch.randn(1, 1, L, D, generator=g, dtype=torch.float64) * valid for _ in range(4))
    rng = np.random.default_rng(8)
    a = rng.random((1, 1, NB, NB)) < 0.2
    ab = a | (rng.random((1, 1, NB, NB)) < 0.35)
    a[:, :, 3] = False
    ab[:, :, 5] = True
    if kmeans:
        km, vm, _, _, lab = ref.kmeans_tables(k.numpy(), v.numpy(), cnt, RM, 5, 3)
        groups = np.where(lab[0, 0] >= 0, (np.arange(L) // 64) * RM + lab[0, 0], -1)
    else:
        km, vm, _, _, _, _ = ref.rep_tables(k.numpy(), v.numpy(), cnt, RM, rnd=lambda x: x)
        lab, groups = None, ref.contiguous_groups(cnt, RM)
    _, _, kt, vt, _, _ = ref.rep_tables(k.numpy(), v.numpy(), cnt, RM, rnd=lambda x: x)
    tables = (km, vm, kt, vt)
    x = [t.clone().requires_grad_(True) for t in (q, k, v)]
    wo, wl = ref.rep_fine_torch(*x, cnt, a, ab, RM, tables=tables, labels=lab)
    wg = torch.autograd.grad(wo, x, do)
    got = ref.rep_fine_head(q[0, 0].numpy(), k[0, 0].numpy(), v[0, 0].numpy(), cnt, a[0, 0], ab[0, 0], RM,
                            [t[0, 0] for t in tables], groups, do[0, 0].numpy())
    assert np.allclose(got["o"], wo.detach().numpy()[0, 0], atol=1e-12)
    fin = np.isfinite(wl.detach().numpy()[0, 0])
    assert np.array_equal(np.isfinite(got["lse"]), fin)
    assert np.allclose(got["lse"][fin], wl.detach().numpy()[0, 0][fin], atol=1e-12)
    for name, w in zip(("dq", "dk", "dv"), wg):
        assert np.allclose(got[name], w.numpy()[0, 0], atol=1e-10), name
        assert (got[name + "_abs"] >= np.abs(got[name]) - 1e-12).all(), name
    # delta from a stored O that differs by eps: delta grows by shift = eps * rowsum(dO), and the gradients are
    # those of sum(O * dO) - sum(shift * lse), since d lse / d s = P
    x2 = [t.clone().requires_grad_(True) for t in (q, k, v)]
    wo2, wl2 = ref.rep_fine_torch(*x2, cnt, a, ab, RM, tables=tables, labels=lab)
    shift = torch.as_tensor((do[0, 0].numpy() * 1e-3).sum(1))
    lse_fin = torch.where(torch.as_tensor(fin), wl2[0, 0], torch.zeros_like(wl2[0, 0]))
    wg2 = torch.autograd.grad((wo2 * do).sum() - (shift * lse_fin).sum(), x2)
    got2 = ref.rep_fine_head(q[0, 0].numpy(), k[0, 0].numpy(), v[0, 0].numpy(), cnt, a[0, 0], ab[0, 0], RM,
                             [t[0, 0] for t in tables], groups, do[0, 0].numpy(),
                             o_delta=wo.detach().numpy()[0, 0] + 1e-3)
    for name, w in zip(("dq", "dk", "dv"), wg2):
        assert np.allclose(got2[name], w.numpy()[0, 0], atol=1e-10), name
    assert np.abs(got2["dq"] - got["dq"]).max() > 1e-6


@pytest.mark.parametrize("kmeans", [False, True])
def test_rep_kv_block_grads_equal_the_head_gradients(kmeans):
    """The per-kv-block gradients from the backward's inputs (LSE, delta) equal the whole-head computation's rows,
    for every block (full, partial, single-token with empty groups)."""
    cnt = [64, 64, 37, 64, 1, 64, 20, 50]
    NB, RM, D = len(cnt), 4, 16
    L = NB * 64
    rng = np.random.default_rng(11)
    valid = ref.token_valid(cnt, L)[:, None]
    q, k, v, do = (rng.standard_normal((L, D)) * valid for _ in range(4))
    a = rng.random((NB, NB)) < 0.2
    ab = a | (rng.random((NB, NB)) < 0.35)
    a[3] = False
    ab[5] = True
    if kmeans:
        km, vm, _, _, lab = ref.kmeans_tables(k[None, None], v[None, None], cnt, RM, 5, 3)
        groups = np.where(lab[0, 0] >= 0, (np.arange(L) // 64) * RM + lab[0, 0], -1)
    else:
        km, vm, _, _, _, _ = ref.rep_tables(k[None, None], v[None, None], cnt, RM, rnd=lambda x: x)
        groups = ref.contiguous_groups(cnt, RM)
    _, _, kt, vt, _, _ = ref.rep_tables(k[None, None], v[None, None], cnt, RM, rnd=lambda x: x)
    tables = [t[0, 0] for t in (km, vm, kt, vt)]
    head = ref.rep_fine_head(q, k, v, cnt, a, ab, RM, tables, groups, do)
    delta = (do * head["o"]).sum(1)
    for j in range(NB):
        got = ref.rep_kv_block_grads(q, k, v, do, head["lse"], delta, cnt, a, ab, j, RM, tables, groups)
        for name in ("dk", "dv", "dk_abs", "dv_abs"):
            assert np.allclose(got[name], head[name][j * 64:(j + 1) * 64], atol=1e-10), (name, j)


def test_rep_tables_counts():
    cnt = [64, 20, 1]
    x = np.random.default_rng(4).standard_normal((1, 1, 192, 8)).astype(np.float32)
    km, vm, kt, vt, lcm, lct = ref.rep_tables(x, x, cnt, 4)
    assert np.allclose(lcm, np.log2([16, 16, 16, 16, 16, 4, 1, 1, 1, 1, 1, 1])[:12].clip(0) * 0 +
                       np.array([4, 4, 4, 4, 4, 2, -np.inf, -np.inf, 0, -np.inf, -np.inf, -np.inf]))
    assert np.allclose(lct, np.log2(cnt))
    assert np.array_equal(km, vm) and (km[0, 0, 6] == 0).all()


def test_blockwise_port_matches_fine_attention():
    cnt = [64, 40, 64, 9]
    q, k, v = (x.numpy().astype(np.float32) for x in _inputs(5, cnt))
    m = np.random.default_rng(6).random((1, 2, 4, 4)) < 0.5
    m[:, :, 2] = False
    ptr, idx = ref.csr_from_mask(m)
    wo, wl = ref.fine_attention(q, k, v, cnt, m)
    for bh in range(2):
        o, lse = ref.fine_attention_blocks(q[0], k[0], v[0], cnt, ptr, idx, bh, range(4))
        assert np.allclose(o.reshape(256, -1), wo[0, bh], atol=1e-5)
        fin = np.isfinite(wl[0, bh])
        assert np.array_equal(np.isfinite(lse.reshape(-1)), fin)
        assert np.allclose(lse.reshape(-1)[fin], wl[0, bh][fin], atol=1e-5)


# --------------------------------------------------------------------------- seeded k-means tables, row tiers
def test_kmeans_seed_tokens():
    """Distinct tokens of the block, min(RM, n) of them, a pure function of (seed, bh, blk), and the seed matters."""
    for n in (1, 3, 4, 20, 64):
        for bh, blk in ((0, 0), (3, 17), (47, 1856)):
            s = ref.kmeans_seed_tokens(7, bh, blk, n, 4)
            assert len(s) == min(4, n) and len(set(s)) == len(s) and all(0 <= t < n for t in s)
            assert s == ref.kmeans_seed_tokens(7, bh, blk, n, 4)
    draws = {tuple(ref.kmeans_seed_tokens(seed, 0, 0, 64, 4)) for seed in range(20)}
    assert len(draws) >= 18


def test_kmeans_tables_invariants():
    """Counts partition each block's valid tokens; every label names a non-empty cluster; each table row is the
    bf16-rounded float64 mean of its members (k and v); empty clusters have zero rows and -inf counts."""
    cnt = [64, 64, 37, 1, 3, 50]
    g = np.random.default_rng(5)
    L, D = len(cnt) * 64, 16
    valid = ref.token_valid(cnt, L)[None, None, :, None]
    k = round_bf16(g.standard_normal((1, 2, L, D)).astype(np.float32)) * valid
    v = round_bf16(g.standard_normal((1, 2, L, D)).astype(np.float32)) * valid
    km, vm, lc, counts, labels = ref.kmeans_tables(k, v, cnt, 4, iters=5, seed=3)
    for bh in range(2):
        for blk, n in enumerate(cnt):
            lab = labels[0, bh, blk * 64:blk * 64 + 64]
            assert (lab[:n] >= 0).all() and (lab[n:] == -1).all()
            c = counts[0, bh, blk * 4:blk * 4 + 4]
            assert c.sum() == n and np.array_equal(c, np.bincount(lab[:n], minlength=4))
            for r in range(4):
                row = blk * 4 + r
                if c[r] == 0:
                    assert np.isneginf(lc[0, bh, row]) and (km[0, bh, row] == 0).all()
                    continue
                assert lc[0, bh, row] == np.log2(c[r])
                members = np.nonzero(lab[:n] == r)[0] + blk * 64
                for tab, x in ((km, k), (vm, v)):
                    want = x[0, bh, members].astype(np.float64).mean(0)
                    assert np.allclose(tab[0, bh, row], want, rtol=2 ** -7, atol=1e-6)
    # a block of n < 4 tokens: every token is its own cluster
    assert np.array_equal(counts[0, 0, 12:16], [1, 0, 0, 0]) and sorted(counts[0, 0, 16:20]) == [0, 1, 1, 1]


def test_kmeans_tables_equal_sklearn_lloyd_from_the_same_seeds():
    """The rounds of kmeans_tables are plain Lloyd iterations: scikit-learn's Lloyd k-means started from the same
    seed tokens and run for the same number of rounds ends at the same centroids (float64 there, float32 here) and
    the same clusters, on blocks of four well-separated groups and on unstructured ones."""
    from sklearn.cluster import KMeans
    g = np.random.default_rng(9)
    D, checked = 32, 0
    for trial in range(24):
        n = 64 - 7 * (trial % 4)
        if trial % 2:
            centers = g.standard_normal((4, D)) * 4
            x = centers[g.integers(0, 4, n)] + 0.3 * g.standard_normal((n, D))
        else:
            x = g.standard_normal((n, D))
        x = round_bf16(x.astype(np.float32))
        k = np.zeros((1, 1, 64, D), np.float32)
        k[0, 0, :n] = x
        km, _, _, counts, labels = ref.kmeans_tables(k, k, [n], 4, iters=5, seed=trial)
        if (counts == 0).any():
            continue   # scikit-learn relocates emptied clusters; the tables keep them empty
        seeds = ref.kmeans_seed_tokens(trial, 0, 0, n, 4)
        sk = KMeans(n_clusters=4, init=x[seeds].astype(np.float64), n_init=1, max_iter=5, tol=0.0,
                    algorithm="lloyd").fit(x.astype(np.float64))
        # scikit-learn's labels_ come from one more assignment against the final centroids; compare partitions
        # through the centroids, which both sides take from the same (last) assignment
        assert np.allclose(km[0, 0], round_bf16(sk.cluster_centers_.astype(np.float32)), rtol=2 ** -7, atol=1e-6)
        checked += 1
    assert checked >= 16


def test_row_tiers_counts_and_nesting():
    """Exactly min(ka, NB) tier-A and min(kab, NB) tier-A|B blocks per row, A inside A|B, and the selection is the
    best-scoring blocks of the row (ties to the smaller index) on a matrix with heavy ties and -0 / +0."""
    g = np.random.default_rng(2)
    s = (g.integers(0, 6, size=(1, 2, 30, 30)) / 5).astype(np.float32)
    s[0, 0, 3, :10] = -0.0
    s[0, 0, 3, 10:] = 0.0
    a, ab = ref.row_tiers(s, 2, 8)
    assert (a.sum(-1) == 2).all() and (ab.sum(-1) == 8).all() and not (a & ~ab).any()
    assert np.array_equal(np.nonzero(a[0, 0, 3])[0], [0, 1])       # -0 == +0: the smaller indices win
    for r in range(30):
        row = s[0, 1, r].astype(np.float64)
        order = sorted(range(30), key=lambda j: (-row[j], j))
        assert np.array_equal(np.nonzero(ab[0, 1, r])[0], sorted(order[:8]))
    a, ab = ref.row_tiers(s, 40, 50)
    assert a.all() and ab.all()
