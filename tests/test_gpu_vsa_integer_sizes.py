"""Byte-for-byte parity of the VSA integer kernels with the oracle on the reference's own edge matrix and at the
sizes the benchmark configurations run:

* the exact global top-k (`vsa_global_topk`: radix select, per-row counts, scan, emission, kv->q inversion) on the
  reference's matrix nb in {1, 7, 33, 130}, with and without ties, budgets {0, 1, nb, 3 nb, nb^2 - 1, nb^2,
  nb^2 + 5} (reference tests/test_vsa2.py:113-144);
* the three-tier routing at C4 (B = 2, H = 24, NB = 1857, 59 bitmap words per row) in both constructions: the
  reference's two global budgets (`vsa_global_topk` twice over one score matrix, with bitmaps) and the
  benchmark's per-query-block split (`vsa_row_tiers`), plus the tier-B lists (`vsa_tier_b_lists`) and the
  transposed tier-A lists, every (b, h) of the launch compared on sampled heads against the oracle's order over
  the same fp32 scores;
* the split-KV planner (`vsa_split_plan`) on the reference's skewed masks (hot rows, hot columns, both, full,
  random), chunk {1, 2, 3, 64}, slot cap {0, 3, 10, none}, over q->kv and kv->q pointers (reference
  tests/test_vsa2_split.py:24-121), and at C5 (47 280 lists of the benchmark's Zipf lengths) over both
  directions and several policies, with every edge covered by exactly one task;
* the CSR transpose (`vsa_csr_transpose`) at C5.

Expected values come from oracle/vsa_ref.py (stable orders over float64 copies of the scores, the restated
planner, numpy CSR construction); nothing here is compared against another GPU result."""
import sys

import numpy as np
import pytest
import torch

from oracle import vsa_ref as ref

pytestmark = pytest.mark.gpu


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def C():
    from self_trainable_or_free_attn_amd.vsa import _C
    return _C


def head_csr(mask, base):
    """(ptr [NB + 1], idx) of one head's bool mask [NB, NB] with absolute offsets starting at base."""
    counts = mask.sum(1)
    ptr = base + np.concatenate([[0], np.cumsum(counts)])
    return ptr.astype(np.int64), np.nonzero(mask)[1].astype(np.int64)


def check_head(name, ptr, idx, b, h, mask, base):
    """The (b, h) rows of a GPU CSR (ptr [B, H, NB + 1], idx flat) equal the oracle's CSR of `mask`."""
    wp, wi = head_csr(mask, base)
    gp = ptr[b, h].astype(np.int64)
    assert np.array_equal(gp, wp), f"{name}: ptr of (b={b}, h={h}) differs"
    assert np.array_equal(idx[gp[0]:gp[-1]].astype(np.int64), wi), f"{name}: idx of (b={b}, h={h}) differs"


def bitmap(mask):
    """Bool [NB, NB] -> int32 words [NB, ceil(NB / 32)], bit j % 32 of word j // 32 = column j."""
    nb = mask.shape[-1]
    w = (nb + 31) // 32
    m = np.zeros((nb, w * 32), bool)
    m[:, :nb] = mask
    words = (m.reshape(nb, w, 32).astype(np.uint64) << np.arange(32, dtype=np.uint64)).sum(-1)
    return words.astype(np.uint32).view(np.int32)


# ------------------------------------------------------------------------- global top-k, the reference's matrix
@pytest.mark.parametrize("nb", [1, 7, 33, 130])
@pytest.mark.parametrize("ties", [False, True])
def test_global_topk_reference_matrix(dev, nb, ties):
    log("global top-k nb", nb, "ties", ties)
    g = np.random.default_rng(nb + 100 * ties)
    BH = 3
    if ties:
        scores = (g.integers(0, 4, (BH, nb, nb)) / 4.0).astype(np.float32)
    else:
        scores = g.random((BH, nb, nb), dtype=np.float32)
    sd = torch.from_numpy(scores).to(dev)
    for budget in sorted({0, 1, nb, 3 * nb, nb * nb - 1, nb * nb, nb * nb + 5}):
        keff = max(0, min(budget, nb * nb))
        out = [torch.full((1, BH, nb + 1), -7, dtype=torch.int32, device=dev),
               torch.full((max(BH * keff, 1),), -7, dtype=torch.int32, device=dev),
               torch.full((1, BH, nb + 1), -7, dtype=torch.int32, device=dev),
               torch.full((max(BH * keff, 1),), -7, dtype=torch.int32, device=dev)]
        C().global_topk_into(sd, budget, 0, *out)
        qp, qi, kp, ki = (x.cpu().numpy() for x in out)
        want = ref.global_topk_mask(scores.reshape(1, BH, nb, nb), budget)[0]
        for h in range(BH):
            assert int(want[h].sum()) == keff
            check_head(f"q2k nb={nb} budget={budget}", qp, qi, 0, h, want[h], h * keff)
            check_head(f"k2q nb={nb} budget={budget}", kp, ki, 0, h, want[h].T, h * keff)
        assert qp[0, -1, -1] == BH * keff


# ------------------------------------------------------------------------- three-tier routing at C4
C4_GRID = (33, 45, 80)
C4_B, C4_H, C4_D = 2, 24, 128
C4_HEADS = [(0, 0), (0, 17), (1, 5), (1, 23)]


@pytest.fixture(scope="module")
def c4_pools(dev):
    from self_trainable_or_free_attn_amd import synthetic
    log("C4 routing: inputs")
    Lr = C4_GRID[0] * C4_GRID[1] * C4_GRID[2]
    NB = -(-Lr // 64)
    qs, ks = [], []
    for b in range(C4_B):
        qb, kb, _, _ = synthetic.fourier_qkv(C4_GRID, C4_H, C4_D, seed=21 + b, device=dev, pad_to=NB * 64)
        qs.append(qb.permute(1, 0, 2))
        ks.append(kb.permute(1, 0, 2))
    q, k = torch.stack(qs).contiguous(), torch.stack(ks).contiguous()
    del qs, ks
    blk = torch.full((NB,), 64, dtype=torch.int32, device=dev)
    blk[-1] = Lr - 64 * (NB - 1)
    return q, k, blk, NB


def _head_scores(C_, q, k, blk, R, b, h):
    """fp32 router scores of one (b, h) from the same pooling / lse / score kernels the routing runs."""
    qr, kr, _, _, _ = C_.pool_fwd(q, k, k, blk, R)
    lse2 = C_.router_lse(qr, kr, blk, R)
    bh = b * q.shape[1] + h
    return C_.router_scores(qr, kr, lse2, blk, R, 1, bh, 1)[0].cpu().numpy()


@pytest.mark.parametrize("split", ["global", "per_row"])
def test_tier_routing_c4_bit_exact(dev, c4_pools, split):
    from self_trainable_or_free_attn_amd.vsa import rep
    q, k, blk, NB = c4_pools
    tiers = rep.RepTiers(frac_full=0.05, frac_mid=0.20, mid_reps=4, split=split)
    log("C4 routing:", split)
    sel = rep.route_tiers(q, k, blk, tiers, R=16)
    torch.cuda.synchronize()
    ap, ai, kp, ki = (x.cpu().numpy() for x in (sel.q2k_ptr, sel.q2k_idx, sel.k2q_ptr, sel.k2q_idx))
    bp, bi = sel.b_ptr.cpu().numpy(), sel.b_idx.cpu().numpy()
    bits_a, bits_ab = sel.bits_a.cpu().numpy(), sel.bits_ab.cpu().numpy()
    assert bits_a.shape[-1] == 59
    if split == "global":
        ka, kab = tiers.budgets(NB)
        base_a, base_b = ka, kab - ka
    else:
        ka, kab = tiers.row_budgets(NB)
        base_a, base_b = NB * ka, NB * (kab - ka)
    for b, h in C4_HEADS:
        log("C4 routing:", split, "oracle of b", b, "h", h)
        s = _head_scores(C(), q, k, blk, 16, b, h)
        if split == "global":
            order = ref._desc_order(s.reshape(-1))
            ma = np.zeros(NB * NB, bool)
            mab = np.zeros(NB * NB, bool)
            ma[order[:ka]] = True
            mab[order[:kab]] = True
            ma, mab = ma.reshape(NB, NB), mab.reshape(NB, NB)
        else:
            ma, mab = ref.row_tiers(s, ka, kab)
            assert (ma.sum(1) == ka).all() and (mab.sum(1) == kab).all()
        bh = b * C4_H + h
        assert np.array_equal(bits_a[b, h], bitmap(ma)), f"tier-A bitmap of (b={b}, h={h}) differs"
        assert np.array_equal(bits_ab[b, h], bitmap(mab)), f"tier-A|B bitmap of (b={b}, h={h}) differs"
        check_head("tier A q2k", ap, ai, b, h, ma, bh * base_a)
        check_head("tier A k2q", kp, ki, b, h, ma.T, bh * base_a)
        check_head("tier B", bp, bi, b, h, mab & ~ma, bh * base_b)


# ------------------------------------------------------------------------- split planner
def skewed_mask(B, H, nb, g, kind):
    """Frozen block masks with skew in the reference's split-plan cases (tests/test_vsa2_split.py:24-48): "hotq"
    a dense row, a mostly dense row, one single-edge row and empty rows; "hotkv" two dense columns over sparse
    random rows with one empty row; "hotqkv" a quarter of the rows 70 % dense plus a dense column and one empty row;
    "full" every pair; "random" 30 % with an empty first row, a dense last row and a single-edge row."""
    m = np.zeros((B, H, nb, nb), bool)
    if kind == "full":
        m[:] = True
    elif kind == "random":
        m = g.random((B, H, nb, nb)) < 0.3
        m[:, :, 0] = False
        m[:, :, -1] = True
        m[:, :, 2] = False
        m[:, :, 2, 1] = True
    elif kind == "hotq":
        m[:, :, 1] = True
        m[:, :, nb - 2] = g.random((B, H, nb)) < 0.8
        m[:, :, 3, 5] = True
    elif kind == "hotkv":
        m = g.random((B, H, nb, nb)) < 2.0 / nb
        m[..., 0] = True
        m[..., nb - 1] = True
        m[:, :, 2] = False
    elif kind == "hotqkv":
        m[:, :, :nb // 4] = g.random((B, H, nb // 4, nb)) < 0.7
        m[..., 1] = True
        m[:, :, nb // 2] = False
    return m


def check_plan(ptr_np, chunk, slots, dev, **policy):
    """GPU plan of the CSR pointers ptr_np against the restated planner, every edge covered by one task."""
    tasks, merges, info = C().split_plan(torch.from_numpy(ptr_np).to(dev), chunk, slots, **policy)
    t_ref, m_ref, i_ref = ref.plan_reference(ptr_np, chunk, slots, **policy)
    assert info.cpu().tolist() == i_ref
    assert tasks[:i_ref[0]].cpu().tolist() == t_ref
    assert merges[:i_ref[1]].cpu().tolist() == m_ref
    lo, hi = int(ptr_np.reshape(-1)[0]), int(ptr_np.reshape(-1)[-1])
    cover = np.zeros(hi - lo + 1, np.int64)
    t = np.asarray(t_ref, np.int64).reshape(-1, 4)
    np.add.at(cover, t[:, 1] - lo, 1)
    np.add.at(cover, t[:, 2] - lo, -1)
    assert (np.cumsum(cover)[:hi - lo] == 1).all(), "an edge is covered by zero or two tasks"
    return i_ref


@pytest.mark.parametrize("kind", ["random", "full", "hotq", "hotkv", "hotqkv"])
@pytest.mark.parametrize("chunk", [1, 2, 3, 64])
def test_split_plan_reference_matrix(dev, kind, chunk):
    from self_trainable_or_free_attn_amd.vsa import ops
    g = np.random.default_rng(chunk)
    nb = 13
    m = skewed_mask(2, 2, nb, g, kind)
    for direction, mm in (("q2k", m), ("k2q", np.swapaxes(m, -1, -2))):
        ptr, idx = ref.csr_from_mask(mm)
        for cap in (0, 3, 10, None):
            slots = ops.split_slots(idx.size, chunk, 1, 1 << 40) if cap is None else cap
            log("split plan", kind, "chunk", chunk, direction, "slots", slots)
            info = check_plan(ptr, chunk, slots, dev)
            assert info[2] <= slots


def c5_mask():
    """The benchmark's C5 selection: H = 40, NB = 1182, per-row counts Zipf(1.2) clipped to [8, 512], columns
    uniform without replacement, seed 4."""
    H, NB = 40, 1182
    rng = np.random.default_rng(4)
    mask = np.zeros((1, H, NB, NB), bool)
    n = np.clip(rng.zipf(1.2, size=(1, H, NB)), 8, 512)
    for h in range(H):
        for i in range(NB):
            mask[0, h, i, rng.choice(NB, size=int(n[0, h, i]), replace=False)] = True
    return mask


@pytest.fixture(scope="module")
def c5():
    log("C5 lists")
    m = c5_mask()
    return m, ref.csr_from_mask(m), ref.csr_from_mask(np.swapaxes(m, -1, -2))


@pytest.mark.parametrize("chunk,slots,policy", [(64, 5000, {}), (64, 1000, {}), (16, 40000, {}),
                                                (64, 100000, dict(min_len=32, rel_mean=4.0, tail_frac=0.0,
                                                                  resident=512, budget=-1)),
                                                (32, 100000, dict(min_len=8, rel_mean=1.5, tail_frac=0.002,
                                                                  resident=512, budget=3000))])
def test_split_plan_c5_bit_exact(dev, c5, chunk, slots, policy):
    _, (qp, _), (kp, _) = c5
    for direction, ptr in (("q2k", qp), ("k2q", kp)):
        log("C5 split plan", direction, "chunk", chunk, "slots", slots, policy)
        info = check_plan(ptr, chunk, slots, dev, **policy)
        assert info[3] == 40 * 1182


def test_csr_transpose_c5(dev, c5):
    _, (qp, qi), (kp, ki) = c5
    log("C5 CSR transpose")
    gp, gi = C().csr_transpose(torch.from_numpy(qp).to(dev), torch.from_numpy(qi).to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(gp.cpu().numpy(), kp)
    assert np.array_equal(gi.cpu().numpy(), ki)
    # and back
    bp, bi = C().csr_transpose(gp, gi)
    assert np.array_equal(bp.cpu().numpy(), qp) and np.array_equal(bi.cpu().numpy(), qi)
