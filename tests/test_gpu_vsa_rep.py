"""Parity of the VSA2 three-tier representative kernels (include/vsa_hip.h, vsa_rep_*) with the CPU oracle
(oracle/vsa_ref.py rep_tables / rep_fine_torch): tables bit for bit (the pooling kernel's float32 order), tier
bitmaps and lists bit for bit on the GPU's own router scores, outputs and gradients at max-abs 2e-2 / rel-L2 1e-2.
Shapes: NB = 10 with partial blocks (one with 1 token, so some representative groups are empty), D = 128."""
import sys

import numpy as np
import pytest
import torch

from helpers import bf16_max_abs, check_close, f32
from oracle import vsa_ref as ref

pytestmark = pytest.mark.gpu

B, H, D = 1, 2, 128
CNT = [64, 64, 37, 64, 1, 64, 64, 20, 64, 50]
NB = len(CNT)
L = NB * 64


def C():
    from self_trainable_or_free_attn_amd.vsa import _C
    return _C


def rep():
    from self_trainable_or_free_attn_amd.vsa import rep as r
    return r


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def tokens(seed, dev, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, H, L, D, generator=g) * scale
    x = (x * torch.as_tensor(ref.token_valid(CNT, L))[None, None, :, None]).to(torch.bfloat16)
    return x, x.to(dev)


@pytest.fixture(scope="module")
def qkv(dev):
    out = [tokens(s, dev) for s in (1, 2, 3)]
    return dict(cpu=[o[0] for o in out], gpu=[o[1] for o in out],
                blk=torch.tensor(CNT, dtype=torch.int32, device=dev))


def tier_masks(seed):
    g = np.random.default_rng(seed)
    a = g.random((B, H, NB, NB)) < 0.15
    ab = a | (g.random((B, H, NB, NB)) < 0.3)
    a[:, :, 3] = False            # a row with no tier-A block
    ab[:, :, 5] = True            # a row with no tier-C block
    return a, ab


def selection(a, ab, dev):
    from self_trainable_or_free_attn_amd.vsa import ops
    sa = ops.mask_to_selection(torch.as_tensor(a).to(dev))
    r = rep()
    sel = r.TierSelection(sa.q2k_ptr, sa.q2k_idx, sa.k2q_ptr, sa.k2q_idx, r.pack_bits(torch.as_tensor(a).to(dev)),
                          r.pack_bits(torch.as_tensor(ab).to(dev)))
    return sel.with_tier_b()


@pytest.mark.parametrize("RM", [1, 4, 16])
def test_rep_tables_bit_exact(qkv, RM):
    log("rep_build RM", RM)
    _, k, v = qkv["gpu"]
    km, vm, lcm, kt, vt, lct = C().rep_build(k, v, qkv["blk"], RM)
    wkm, wvm, wkt, wvt, wlcm, wlct = ref.rep_tables(f32(qkv["cpu"][1]), f32(qkv["cpu"][2]), CNT, RM)
    assert np.array_equal(f32(km)[:, :, :NB * RM], wkm) and np.array_equal(f32(vm)[:, :, :NB * RM], wvm)
    assert np.array_equal(f32(kt)[:, :, :NB], wkt) and np.array_equal(f32(vt)[:, :, :NB], wvt)
    # log2 of integer counts: the device log2f is within 2 ulp, not correctly rounded
    gl, gt = lcm.cpu().numpy(), lct.cpu().numpy()
    assert np.array_equal(np.isfinite(gl), np.isfinite(wlcm))
    assert np.allclose(gl[np.isfinite(gl)], wlcm[np.isfinite(wlcm)], rtol=0, atol=2e-6)
    assert np.allclose(gt, wlct, rtol=0, atol=2e-6)


def test_pack_bits_round_trip(dev):
    r = rep()
    m = torch.as_tensor(np.random.default_rng(0).random((1, 2, 45, 45)) < 0.4).to(dev)
    assert torch.equal(r._unpack_bits(r.pack_bits(m), 45), m)


@pytest.mark.parametrize("frac_full,frac_mid", [(0.1, 0.2), (0.15, 0.0), (0.0, 0.5)])
def test_route_tiers_bit_exact(qkv, frac_full, frac_mid):
    log("route_tiers", frac_full, frac_mid)
    q, k, _ = qkv["gpu"]
    r = rep()
    tiers = r.RepTiers(frac_full=frac_full, frac_mid=frac_mid)
    sel = r.route_tiers(q, k, qkv["blk"], tiers, R=16)
    qr, kr, _, _, _ = C().pool_fwd(q, k, k, qkv["blk"], 16)
    lse2 = C().router_lse(qr, kr, qkv["blk"], 16)
    s = f32(C().router_scores(qr, kr, lse2, qkv["blk"], 16, 1)).reshape(B, H, NB, NB)
    ba, bab = tiers.budgets(NB)
    wa, wab = ref.global_topk_mask(s, ba), ref.global_topk_mask(s, bab)
    a, b, c = (x.cpu().numpy() for x in sel.tier_masks(NB))
    assert np.array_equal(a, wa) and np.array_equal(a | b, wab) and np.array_equal(c, ~wab)
    rp, ri = ref.csr_from_mask(wa)
    assert np.array_equal(sel.q2k_ptr.cpu().numpy(), rp) and np.array_equal(sel.q2k_idx.cpu().numpy()[:ri.size], ri)
    bp, bi = ref.csr_from_mask(wab & ~wa)
    assert np.array_equal(sel.b_ptr.cpu().numpy(), bp)
    assert np.array_equal(sel.b_idx.cpu().numpy()[:bi.size], bi)


@pytest.mark.parametrize("phases", [7, 1, 2, 4, 6])
@pytest.mark.parametrize("RM", [4, 2])
def test_rep_forward(qkv, phases, RM):
    log("rep fwd phases", phases, "RM", RM)
    q, k, v = qkv["gpu"]
    a, ab = tier_masks(phases + RM)
    sel = selection(a, ab, q.device)
    o, lse = rep().rep_fine_attention(q, k, v, qkv["blk"], sel, mid_reps=RM, phases=phases)
    torch.cuda.synchronize()
    km, vm, kt, vt, _, _ = ref.rep_tables(f32(qkv["cpu"][1]), f32(qkv["cpu"][2]), CNT, RM)
    x = [t.double() for t in qkv["cpu"]]
    wo, wl = ref.rep_fine_torch(*x, CNT, a, ab, RM, phases, tables=(km, vm, kt, vt))
    check_close("O", f32(o), wo.numpy())
    wl = wl.numpy()
    fin = np.isfinite(wl)
    assert np.array_equal(np.isfinite(f32(lse)), fin)
    check_close("lse", f32(lse)[fin], wl[fin])


@pytest.mark.parametrize("phases", [7, 6, 1])
def test_rep_backward(qkv, phases):
    log("rep bwd phases", phases)
    RM = 4
    q, k, v = (t.detach().clone().requires_grad_(True) for t in qkv["gpu"])
    a, ab = tier_masks(30 + phases)
    sel = selection(a, ab, q.device)
    o, _ = rep().rep_fine_attention(q, k, v, qkv["blk"], sel, mid_reps=RM, phases=phases)
    dout_c, dout = tokens(40, q.device)
    grads = torch.autograd.grad(o, (q, k, v), dout)
    torch.cuda.synchronize()
    km, vm, kt, vt, _, _ = ref.rep_tables(f32(qkv["cpu"][1]), f32(qkv["cpu"][2]), CNT, RM)
    x = [t.double().requires_grad_(True) for t in qkv["cpu"]]
    wo, _ = ref.rep_fine_torch(*x, CNT, a, ab, RM, phases, tables=(km, vm, kt, vt))
    wg = torch.autograd.grad(wo, x, dout_c.double())
    for name, g, w in zip(("dQ", "dK", "dV"), grads, wg):
        check_close(name, f32(g), w.numpy(), max_abs=bf16_max_abs(w.numpy()))


def test_rep_attention_end_to_end(qkv):
    log("rep_attention")
    r = rep()
    q, k, v = (t.detach().clone().requires_grad_(True) for t in qkv["gpu"])
    g = torch.Generator().manual_seed(50)
    gate_c = torch.randn(B, H, L, generator=g).to(torch.bfloat16)
    gate = gate_c.to(q.device).requires_grad_(True)
    tiers = r.RepTiers(frac_full=0.1, frac_mid=0.2)
    o, sel = r.rep_attention(q, k, v, gate, qkv["blk"], R=16, tiers=tiers, return_selection=True)
    dout_c, dout = tokens(51, q.device)
    grads = torch.autograd.grad(o, (q, k, v, gate), dout)
    a, b, _ = (m.cpu().numpy() for m in sel.tier_masks(NB))
    ab = a | b
    assert a.sum() == B * H * tiers.budgets(NB)[0] and ab.sum() == B * H * tiers.budgets(NB)[1]
    # oracle: three-tier fine branch + coarse branch + gate, with the kernels' bf16 tables and block means
    km, vm, kt, vt, _, _ = ref.rep_tables(f32(qkv["cpu"][1]), f32(qkv["cpu"][2]), CNT, 4)
    _, _, qc, kc, vc = C().pool_fwd(*qkv["gpu"], qkv["blk"], 16)
    x = [t.double().requires_grad_(True) for t in (*qkv["cpu"], gate_c)]
    fine, _ = ref.rep_fine_torch(*x[:3], CNT, a, ab, 4, 7, tables=(km, vm, kt, vt))
    coarse_only = ref.vsa_output(*x[:3], x[3], CNT, np.zeros_like(a), "tanh",
                                 pooled=[f32(t)[:, :, :NB] for t in (qc, kc, vc)])
    want = fine + coarse_only
    wg = torch.autograd.grad(want, x, dout_c.double())
    check_close("O", f32(o), want.detach().numpy())
    for name, gr, w in zip(("dQ", "dK", "dV", "dgate"), grads, wg):
        wn = w.numpy()
        check_close(name, f32(gr), wn, max_abs=bf16_max_abs(wn))


# ------------------------------------------------- the three-tier benchmark construction: k-means tables, per-row tiers
@pytest.mark.parametrize("RM,seed", [(4, 0), (4, 11), (1, 3), (16, 5)])
def test_kmeans_tables_bit_exact(qkv, RM, seed):
    """vsa_rep_build_kmeans against oracle kmeans_tables: tables, cluster sizes and labels equal bit for bit (the
    kernel restates the float32 order with no fused multiply-add); the tail tables are rep_build's."""
    log("kmeans tables RM", RM, "seed", seed)
    _, k, v = qkv["gpu"]
    tab, counts, labels = C().rep_build_kmeans(k, v, qkv["blk"], RM, iters=5, seed=seed)
    torch.cuda.synchronize()
    wkm, wvm, wlc, wcnt, wlab = ref.kmeans_tables(f32(qkv["cpu"][1]), f32(qkv["cpu"][2]), CNT, RM, 5, seed)
    assert np.array_equal(counts.cpu().numpy(), wcnt)
    lab = labels.cpu().numpy().astype(np.int64)
    assert np.array_equal(np.where(lab == 255, -1, lab), wlab)
    assert np.array_equal(f32(tab[0])[:, :, :NB * RM], wkm) and np.array_equal(f32(tab[1])[:, :, :NB * RM], wvm)
    gl = tab[2].cpu().numpy()
    assert gl.shape == (B, H, NB * RM) and np.array_equal(np.isfinite(gl), np.isfinite(wlc))
    assert np.allclose(gl[np.isfinite(gl)], wlc[np.isfinite(wlc)], rtol=0, atol=2e-6)
    _, _, kt, vt, _, _ = ref.rep_tables(f32(qkv["cpu"][1]), f32(qkv["cpu"][2]), CNT, RM)
    assert np.array_equal(f32(tab[3])[:, :, :NB], kt) and np.array_equal(f32(tab[4])[:, :, :NB], vt)
    if RM == 4:  # the seed changes the clustering of at least one block
        _, c2, _ = C().rep_build_kmeans(k, v, qkv["blk"], RM, iters=5, seed=seed + 1)
        assert not torch.equal(c2, counts)


@pytest.mark.parametrize("frac_full,frac_mid", [(0.05, 0.20), (0.3, 0.0), (0.0, 0.5), (1.0, 0.0)])
def test_row_tiers_bit_exact(qkv, frac_full, frac_mid):
    """The per-row tier split on the GPU's own router scores: bitmaps, tier-A lists, their transpose and the tier-B
    lists equal the oracle's (row_topk order: score desc, ties to the smaller index)."""
    log("row tiers", frac_full, frac_mid)
    q, k, _ = qkv["gpu"]
    r = rep()
    tiers = r.RepTiers(frac_full=frac_full, frac_mid=frac_mid, split="per_row")
    sel = r.route_tiers(q, k, qkv["blk"], tiers, R=16)
    qr, kr, _, _, _ = C().pool_fwd(q, k, k, qkv["blk"], 16)
    lse2 = C().router_lse(qr, kr, qkv["blk"], 16)
    s = f32(C().router_scores(qr, kr, lse2, qkv["blk"], 16, 1)).reshape(B, H, NB, NB)
    ka, kab = tiers.row_budgets(NB)
    wa, wab = ref.row_tiers(s, ka, kab)
    a, b, c = (x.cpu().numpy() for x in sel.tier_masks(NB))
    assert np.array_equal(a, wa) and np.array_equal(a | b, wab) and np.array_equal(c, ~wab)
    rp, ri = ref.csr_from_mask(wa)
    assert np.array_equal(sel.q2k_ptr.cpu().numpy(), rp) and np.array_equal(sel.q2k_idx.cpu().numpy()[:ri.size], ri)
    tp, ti = ref.csr_from_mask(np.swapaxes(wa, 2, 3))
    assert np.array_equal(sel.k2q_ptr.cpu().numpy(), tp) and np.array_equal(sel.k2q_idx.cpu().numpy()[:ti.size], ti)
    bp, bi = ref.csr_from_mask(wab & ~wa)
    assert np.array_equal(sel.b_ptr.cpu().numpy(), bp) and np.array_equal(sel.b_idx.cpu().numpy()[:bi.size], bi)


def _kmeans_ref_tables(qkv, RM, seed):
    km, vm, _, _, lab = ref.kmeans_tables(f32(qkv["cpu"][1]), f32(qkv["cpu"][2]), CNT, RM, 5, seed)
    _, _, kt, vt, _, _ = ref.rep_tables(f32(qkv["cpu"][1]), f32(qkv["cpu"][2]), CNT, RM)
    return (km, vm, kt, vt), lab


@pytest.mark.parametrize("phases", [7, 2, 6])
def test_rep_forward_backward_kmeans_tables(qkv, phases):
    """The three-tier attention over k-means tables (per-head log2 cluster sizes, gradients spread over the
    clusters) against the float64 graph whose representatives are the clusters' means."""
    log("rep kmeans fwd+bwd phases", phases)
    RM, seed = 4, 2
    q, k, v = (t.detach().clone().requires_grad_(True) for t in qkv["gpu"])
    a, ab = tier_masks(60 + phases)
    sel = selection(a, ab, q.device)
    o, lse = rep().rep_fine_attention(q, k, v, qkv["blk"], sel, mid_reps=RM, phases=phases, tables="kmeans",
                                      kmeans_iters=5, seed=seed)
    dout_c, dout = tokens(41, q.device)
    grads = torch.autograd.grad(o, (q, k, v), dout)
    torch.cuda.synchronize()
    tables, lab = _kmeans_ref_tables(qkv, RM, seed)
    x = [t.double().requires_grad_(True) for t in qkv["cpu"]]
    wo, wl = ref.rep_fine_torch(*x, CNT, a, ab, RM, phases, tables=tables, labels=lab)
    check_close("O", f32(o), wo.detach().numpy())
    wl = wl.detach().numpy()
    fin = np.isfinite(wl)
    assert np.array_equal(np.isfinite(f32(lse)), fin)
    check_close("lse", f32(lse)[fin], wl[fin])
    wg = torch.autograd.grad(wo, x, dout_c.double())
    for name, g, w in zip(("dQ", "dK", "dV"), grads, wg):
        check_close(name, f32(g), w.numpy(), max_abs=bf16_max_abs(w.numpy()))


def test_rep_attention_config4_construction(qkv):
    """rep_attention as the three-tier benchmark states it: per-row tiers (5 % / 20 %) and seeded 5-round k-means tables,
    forward and backward against the float64 graph on the same selection and clusters."""
    log("rep_attention per_row + kmeans")
    r = rep()
    q, k, v = (t.detach().clone().requires_grad_(True) for t in qkv["gpu"])
    tiers = r.RepTiers(frac_full=0.2, frac_mid=0.3, split="per_row", tables="kmeans", seed=7)
    o, sel = r.rep_attention(q, k, v, None, qkv["blk"], R=16, tiers=tiers, return_selection=True)
    dout_c, dout = tokens(52, q.device)
    grads = torch.autograd.grad(o, (q, k, v), dout)
    a, b, _ = (m.cpu().numpy() for m in sel.tier_masks(NB))
    ka, kab = tiers.row_budgets(NB)
    assert (a.sum(-1) == ka).all() and ((a | b).sum(-1) == kab).all()
    tables, lab = _kmeans_ref_tables(qkv, 4, 7)
    _, _, qc, kc, vc = C().pool_fwd(*qkv["gpu"], qkv["blk"], 16)
    x = [t.double().requires_grad_(True) for t in qkv["cpu"]]
    fine, _ = ref.rep_fine_torch(*x, CNT, a, a | b, 4, 7, tables=tables, labels=lab)
    coarse = ref.vsa_output(*x, None, CNT, np.zeros_like(a), "tanh",
                            pooled=[f32(t)[:, :, :NB] for t in (qc, kc, vc)])
    want = fine + coarse
    wg = torch.autograd.grad(want, x, dout_c.double())
    check_close("O", f32(o), want.detach().numpy())
    for name, gr, w in zip(("dQ", "dK", "dV"), grads, wg):
        wn = w.numpy()
        check_close(name, f32(gr), wn, max_abs=bf16_max_abs(wn))
