"""Pins of the CPU oracle (oracle/echosparse_ref.py) against definitions that do not share its code: torch softmax /
logsumexp attention, brute-force scalar loops on tiny inputs, the reference's literal 31-step bisection, hand-made
known answers for the block selection, and algebraic invariants of the representatives. CPU only."""
import math

import numpy as np
import pytest
import torch

from helpers import structured_qkv
from oracle import echosparse_ref as ref
from oracle.bf16 import from_bf16_bits, round_bf16, to_bf16_bits

LN2 = math.log(2.0)


def qkv(L, H, seed=0):
    (q, k, v), = structured_qkv(L, H, seed=seed)
    return q.float().numpy(), k.float().numpy(), v.float().numpy()


def torch_attention(q, k, v, keys, bias=None):
    """softmax(q k^T / sqrt(D) + bias) v over the given key rows, natural units; returns (O, natural LSE)."""
    qt, kt, vt = (torch.from_numpy(np.asarray(x, np.float64)) for x in (q, k[keys], v[keys]))
    s = qt @ kt.T / math.sqrt(q.shape[-1])
    if bias is not None:
        s = s + torch.from_numpy(np.asarray(bias, np.float64))[None, :]
    return (torch.softmax(s, -1) @ vt).numpy(), torch.logsumexp(s, -1).numpy()


# ------------------------------------------------------------------------------------------------- bf16
def test_round_bf16_matches_torch():
    g = np.random.default_rng(0)
    x = np.concatenate([g.standard_normal(10000).astype(np.float32) * 10 ** g.uniform(-30, 30, 10000),
                        np.array([1.00390625, 1.01171875, -1.00390625, 3.0e-39, 65504.0, np.inf, -np.inf],
                                 np.float32)]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(round_bf16(x), want)
    assert np.array_equal(from_bf16_bits(to_bf16_bits(x)), want)


# ------------------------------------------------------------------------------ fixed-offset attention
def test_fixed_offset_attention_all_blocks_is_dense_attention():
    L, H = 700, 2             # 11 kv blocks (tail 60), 6 query tiles (tail 60)
    q, k, v = qkv(L, H)
    nq, nb = ref.cdiv(L, 128), ref.cdiv(L, 64)
    allb = np.broadcast_to(np.arange(nb, dtype=np.int32), (nq, H, nb))
    cnt = np.full((nq, H), nb, np.int32)
    prior = np.random.default_rng(1).normal(0, 3, (nq * 128, H)).astype(np.float32)
    out, lse, flags, mass = ref.fixed_offset_attention(q, k, v, cnt, allb, prior, threshold=1e9, write_mass=True)
    for h in range(H):
        o, lse_nat = torch_attention(q[:, h], k[:, h], v[:, h], np.arange(L))
        assert np.allclose(out[:, h], o, atol=1e-9)
        # LSE = prior + log2(sum 2^(s*log2e - prior)) = natural LSE / ln 2
        assert np.allclose(lse[:L, h], lse_nat / LN2, atol=1e-9)
    assert (lse[L:] == 1e30).all() and not flags.any()
    # the masses of a tile's blocks add up to its row sums 2^(LSE - prior)
    rows = np.exp2(lse[:L] - prior[:L])
    for t in range(nq):
        r0, r1 = t * 128, min(L, t * 128 + 128)
        assert np.allclose(mass[:, t].sum(-1), rows[r0:r1].sum(0), rtol=1e-9)


def test_mass_map_brute_force():
    """mass[h, t, b] = sum over the tile's valid rows and b's valid keys of 2^(q.k log2e/sqrt(D) - prior)."""
    L, H, D = 200, 1, 128
    q, k, v = qkv(L, H, seed=3)
    nq, nb = ref.cdiv(L, 128), ref.cdiv(L, 64)
    prior = np.full((nq * 128, H), 1e30, np.float32)
    prior[:L, 0] = np.linspace(5, 9, L)
    blocks = np.array([[[2, 0, 3]], [[1, 3, 0]]], np.int32)
    counts = np.array([[2], [3]], np.int32)
    _, _, _, mass = ref.fixed_offset_attention(q, k, v, counts, blocks, prior, threshold=1e9, write_mass=True)
    c = math.log2(math.e) / math.sqrt(D)
    for t in range(nq):
        for b in range(nb):
            listed = b in blocks[t, 0, :counts[t, 0]]
            want = 0.0
            if listed:
                for r in range(t * 128, min(L, t * 128 + 128)):
                    for j in range(b * 64, min(L, b * 64 + 64)):
                        want += 2.0 ** (float(np.dot(q[r, 0].astype(np.float64), k[j, 0])) * c - float(prior[r, 0]))
            assert math.isclose(mass[0, t, b], want, rel_tol=1e-9, abs_tol=0.0)


def test_offset_cancels_in_output():
    L, H = 500, 1
    q, k, v = qkv(L, H, seed=2)
    nq, nb = ref.cdiv(L, 128), ref.cdiv(L, 64)
    blocks = np.tile(np.array([0, 3, 5, 7], np.int32), (nq, H, 1))
    counts = np.full((nq, H), 4, np.int32)
    p1 = np.zeros((nq * 128, H), np.float32)
    p2 = np.random.default_rng(0).normal(0, 20, p1.shape).astype(np.float32)
    o1, l1, _, _ = ref.fixed_offset_attention(q, k, v, counts, blocks, p1)
    o2, l2, _, _ = ref.fixed_offset_attention(q, k, v, counts, blocks, p2)
    assert np.allclose(o1, o2, atol=1e-9) and np.allclose(l1[:L], l2[:L], atol=1e-9)


def sparse_case(L=4152, H=1, seed=0, density=0.1):
    """A plan, block means and representatives for a sparse step (oracle-made, structured inputs)."""
    q, k, v = qkv(L, H, seed=seed)
    nq, nb = ref.cdiv(L, 128), ref.cdiv(L, 64)
    allb = np.broadcast_to(np.arange(nb, dtype=np.int32), (nq, H, nb))
    cnt = np.full((nq, H), nb, np.int32)
    _, lse0, _, _ = ref.fixed_offset_attention(q, k, v, cnt, allb, np.zeros((nq * 128, H), np.float32))
    prior = lse0.astype(np.float32)
    _, lse, flags, mass = ref.fixed_offset_attention(q, k, v, cnt, allb, prior, write_mass=True)
    se, ss = ref.full_step_scales(prior, lse.astype(np.float32), L)
    top, refined = ref.budget(density, nb)
    rw, words = -(-refined // 32) * 32, ref.plan_words(nb)
    keep, counts, blocks, refine, skip = ref.select_blocks(mass.astype(np.float32), np.ones((H, nq, nb), np.uint8),
                                                           se.astype(np.float32), ss.astype(np.float32), flags,
                                                           top, refined, L, rw, words)
    lists = ref.rebuild_plan(ref.pack_plan(keep, words), skip, nb, rw)
    km, vm = ref.block_means(k, v)
    kr, vr, lc = ref.representatives(q, k, v, iters=6)
    comp = dict(k_mean=km, v_mean=vm, means=lists[5], mean_counts=lists[6], refine=lists[3], refine_counts=lists[4],
                k_rep=kr, v_rep=vr, log_counts=lc)
    return q, k, v, prior, lists, comp


def test_sparse_step_matches_explicit_formula():
    """The reference's check_formula (tests/test_attention.py:72-100): exact tokens of the listed blocks, block means
    of the other skipped blocks (+ ln block length), four representatives of each refined block (+ ln count), all
    in one softmax -- restated with torch in natural units."""
    L = 4152
    q, k, v, prior, lists, comp = sparse_case(L)
    keep, counts, blocks, refine, rc, means, mc = lists
    out, _, _, _ = ref.fixed_offset_attention(q, k, v, counts, blocks, prior, comp=comp)
    nb = ref.cdiv(L, 64)
    blen = np.full(nb, 64.0)
    blen[-1] = L - 64 * (nb - 1)
    for t in (0, 7, 32):
        exact = blocks[t, 0, :counts[t, 0]].tolist()
        refined = [b for b in refine[t, 0].tolist() if b < nb]
        mean_ids = sorted(set(range(nb)) - set(exact) - set(refined))
        assert mean_ids == means[t, 0, :mc[t, 0]].tolist()
        rows = np.arange(128 * t, min(128 * t + 128, L))
        keys = [k[64 * b:min(64 * b + 64, L), 0] for b in exact] + [comp["k_mean"][mean_ids, 0]]
        vals = [v[64 * b:min(64 * b + 64, L), 0] for b in exact] + [comp["v_mean"][mean_ids, 0]]
        bias = [np.zeros(min(64 * b + 64, L) - 64 * b) for b in exact] + [np.log(blen[mean_ids])]
        for b in refined:
            keys.append(comp["k_rep"][0, 4 * b:4 * b + 4])
            vals.append(comp["v_rep"][0, 4 * b:4 * b + 4])
            bias.append(comp["log_counts"][0, 4 * b:4 * b + 4].astype(np.float64) * LN2)
        kk, vv, bb = np.concatenate(keys), np.concatenate(vals), np.concatenate(bias)
        s = torch.from_numpy(q[rows, 0].astype(np.float64)) @ torch.from_numpy(kk.astype(np.float64)).T / math.sqrt(128)
        want = (torch.softmax(s + torch.from_numpy(bb)[None], -1) @ torch.from_numpy(vv.astype(np.float64))).numpy()
        assert np.allclose(out[rows, 0], want, atol=1e-9)


def test_fallback_and_compensation_are_one_softmax():
    """exact_fallback = softmax over the listed blocks' tokens; compensate_fallback then appends the mean columns
    of every keep == 0 block (+ ln length) to that softmax (reference triton_ops.py:275-282)."""
    L = 4152
    q, k, v, prior, lists, comp = sparse_case(L, seed=1)
    keep, counts, blocks = lists[:3]
    nq, nb = ref.cdiv(L, 128), ref.cdiv(L, 64)
    out = np.zeros((L, 1, 128))
    lse = np.zeros((nq * 128, 1))
    flags = np.ones((nq, 1), np.int32)
    ref.exact_fallback(q, k, v, out, counts, blocks, lse, flags)
    blen = np.full(nb, 64.0)
    blen[-1] = L - 64 * (nb - 1)
    for t in (1, 20, 32):
        rows = np.arange(128 * t, min(128 * t + 128, L))
        tok = np.concatenate([np.arange(64 * b, min(64 * b + 64, L)) for b in blocks[t, 0, :counts[t, 0]]])
        o, lse_nat = torch_attention(q[rows, 0], k[:, 0], v[:, 0], tok)
        assert np.allclose(out[rows, 0], o, atol=1e-9) and np.allclose(lse[rows, 0], lse_nat / LN2, atol=1e-9)
    km, vm = comp["k_mean"], comp["v_mean"]
    ref.compensate_fallback(q, km, vm, keep, lse, out, flags)
    for t in (1, 20, 32):
        rows = np.arange(128 * t, min(128 * t + 128, L))
        tok = np.concatenate([np.arange(64 * b, min(64 * b + 64, L)) for b in blocks[t, 0, :counts[t, 0]]])
        skipped = np.flatnonzero(keep[0, t] == 0)
        kk = np.concatenate([k[tok, 0], km[skipped, 0]])
        vv = np.concatenate([v[tok, 0], vm[skipped, 0]])
        bb = np.concatenate([np.zeros(tok.size), np.log(blen[skipped])])
        o, lse_nat = torch_attention(q[rows, 0], kk, vv, np.arange(kk.shape[0]), bias=bb)
        assert np.allclose(out[rows, 0], o, atol=1e-9) and np.allclose(lse[rows, 0], lse_nat / LN2, atol=1e-9)


# ---------------------------------------------------------------------------------- selection and plans
def bisection_kth(bits, K):
    """The reference's _kth_largest, step by step (echosparse/kernels/triton_ops.py:43-54), for a brute-force
    cross-check of the oracle's sort-based closed form."""
    lo, hi = 0, 0x7F800001
    bits = np.asarray(bits, np.int64)
    for _ in range(31):
        mid = lo + (hi - lo) // 2
        if int((bits >= mid).sum()) >= K:
            lo = mid
        else:
            hi = mid
    return lo


def test_kth_largest_equals_bisection():
    g = np.random.default_rng(0)
    for trial in range(300):
        n = int(g.integers(1, 40))
        vals = g.choice(np.array([0.0, 0.25, 0.5, 1.0, 3.0, np.inf, -1.0], np.float32), n)
        vals = np.where(g.random(n) < 0.3, g.random(n).astype(np.float32), vals).astype(np.float32)
        bits = vals.view(np.int32)
        for K in range(0, n + 3):
            assert ref.kth_largest_bits(bits, K) == bisection_kth(bits, K), (vals, K)


def test_select_blocks_known_answers():
    """L = 1024: 8 tiles, 16 blocks. Tile t owns blocks 2t, 2t+1; forced = 2t-1 .. 2t+2 (clipped) and >= sink."""
    L, H, nq, nb = 1024, 1, 8, 16
    mass = np.zeros((H, nq, nb), np.float32)
    mass[0, 0] = [0, 0, 0, 0, .5, .5, .5, .2, .9, .1, .1, .1, .3, .3, 0, 0]   # 3-way tie at the 4th value
    mass[0, 3] = [.8, .7, np.nan, .6, .6, .6, .6, .6, .6, .05, .5, .5, .5, 1, 1, 1]
    mass[0, 5] = np.linspace(1, 0, nb)
    keep_prev = np.zeros((H, nq, nb), np.uint8)
    keep_prev[0, 5, [15, 14]] = 1                      # previously kept; tile 5 fell back -> kept first
    se = np.ones((H, nq), np.float32)
    ss = np.ones((H, nq), np.float32)
    flags = np.zeros((nq, H), np.int32)
    flags[5, 0] = 1
    K, R, RW, words = 4, 3, 4, ref.plan_words(nb)
    keep, counts, blocks, refine, skip = ref.select_blocks(mass, keep_prev, se, ss, flags, K, R, L, RW, words)
    # tile 0: forced 0..2 (lo = -1); top-4 values .9, .5, .5, .5 -> every tied .5 kept
    assert blocks[0, 0, :counts[0, 0]].tolist() == [0, 1, 2, 4, 5, 6, 8]
    # refine: largest raw among the rest: .3, .3, .2 -> blocks 12, 13, 7 in block order
    assert refine[0, 0].tolist() == [7, 12, 13, nb]
    # tile 3 (forced 5..8): top-4 = 1, 1, 1, .8; NaN counts as 0
    assert blocks[3, 0, :counts[3, 0]].tolist() == [0, 5, 6, 7, 8, 13, 14, 15]
    # refine: .7, then the ties at .6 (3, 4) cut by block order; R = 3
    assert refine[3, 0].tolist() == [1, 3, 4, nb]
    # tile 5: fell back, so its previously kept 14, 15 are +inf; then 1.0 (block 0) and .93 (1); forced 9..12
    assert blocks[5, 0, :counts[5, 0]].tolist() == [0, 1, 9, 10, 11, 12, 14, 15]
    # skip bits: kept or refined, and every bit >= nb
    for t in range(nq):
        bits = ref._unpack_words(skip[0, t], 32)
        want = np.zeros(32, bool)
        want[:nb] = keep[0, t].astype(bool)
        want[[b for b in refine[t, 0] if b < nb]] = True
        want[nb:] = True
        assert np.array_equal(bits, want)
    # a sink: every block >= sink is forced and +inf
    keep2, counts2, blocks2, *_ = ref.select_blocks(mass, keep_prev, se, ss, flags, K, R, L, RW, words, sink=14)
    # top-4 = inf, inf (14, 15), .9 (8), .5 -> the .5 ties 4, 5, 6 stay in
    assert blocks2[0, 0, :counts2[0, 0]].tolist() == [0, 1, 2, 4, 5, 6, 8, 14, 15]


def test_pack_rebuild_round_trip():
    """select -> pack -> rebuild reproduces keep, the block list and the refine list; the mean list is the
    complement of kept and refined blocks (reference tests/test_sm120.py:109-140)."""
    L, H = 4152, 3
    nq, nb = ref.cdiv(L, 128), ref.cdiv(L, 64)
    g = np.random.default_rng(0)
    mass = g.random((H, nq, nb)).astype(np.float32)
    keep_prev = (g.random((H, nq, nb)) < 0.1).astype(np.uint8)
    ones = np.ones((H, nq), np.float32)
    flags = np.zeros((nq, H), np.int32)
    words = ref.plan_words(nb)
    keep, counts, blocks, refine, skip = ref.select_blocks(mass, keep_prev, ones, ones, flags, 7, 20, L, 32, words,
                                                           sink=60)
    exact = ref.pack_plan(keep, words)
    k2, c2, b2, r2, rc, m2, mc = ref.rebuild_plan(exact, skip, nb, 32)
    assert np.array_equal(k2, keep) and np.array_equal(c2, counts) and np.array_equal(r2, refine)
    assert np.array_equal(b2, blocks)
    assert np.array_equal(rc, (refine < nb).sum(-1))
    for t in range(nq):
        for h in range(H):
            listed = set(blocks[t, h, :counts[t, h]]) | set(refine[t, h][refine[t, h] < nb])
            assert m2[t, h, :mc[t, h]].tolist() == sorted(set(range(nb)) - listed)


def test_plan_word_bit_order_known_value():
    """Bit i of plan word w is block 32 w + i, and the bits of blocks nb..next_pow2(nb) - 1 are set (reference
    echosparse/kernels/sm120.py:258-267): nb = 40 with blocks 0, 5 and 33 kept gives words 0x21 and 0xFFFFFF02;
    the words past next_pow2(nb) / 32 keep the plans' initial -1."""
    keep = np.zeros((1, 1, 40), np.uint8)
    keep[0, 0, [0, 5, 33]] = 1
    words = ref.pack_plan(keep, 4)
    assert words.tolist() == [[[0x21, -254, -1, -1]]]
    assert np.int32(-254).view(np.uint32) == 0xFFFFFF02


def test_budget_known_values():
    assert ref.budget(0.10, 1182) == (118, 355)         # Wan2.1-14B 720p
    assert ref.budget(0.10, 65) == (6, 20)
    assert ref.plan_words(1182) == 64 and ref.plan_words(65) == 4


# ------------------------------------------------------------------------------------- estimate / scales
def test_estimate_brute_force():
    L, H, D = 300, 1, 128                 # 3 tiles (tail 44), 5 blocks (tail 44)
    q, k, v = qkv(L, H, seed=4)
    nq, nb = 3, 5
    km, _ = ref.block_means(k, v)
    g = np.random.default_rng(2)
    keep = (g.random((H, nq, nb)) < 0.5).astype(np.uint8)
    off = np.full((nq * 128, H), 1e30, np.float32)
    off[:L] = g.normal(8, 1, (L, H))
    lse = off.copy()
    lse[:L] += g.normal(0, 0.2, (L, H)).astype(np.float32)
    mass0 = g.random((H, nq, nb)).astype(np.float32) * 10
    mass = mass0.copy()
    se, ss = ref.estimate_skipped(q, km, keep, off, lse, mass)
    c = math.log2(math.e) / math.sqrt(D)
    for t in range(nq):
        rows = [r for r in range(t * 128, t * 128 + 128, 8) if r < L]
        nrows = min(L - t * 128, 128)
        est = []
        for b in range(nb):
            lb = 6.0 if b < nb - 1 else math.log2(L - 64 * (nb - 1))
            e = sum(2.0 ** min(float(np.dot(q[r, 0].astype(np.float64), km[b, 0])) * c - float(off[r, 0]) + lb, 100.0)
                    for r in rows)
            est.append(e / len(rows))
        for b in range(nb):
            want = est[b] if keep[0, t, b] == 0 else float(mass0[0, t, b])
            assert math.isclose(mass[0, t, b], want, rel_tol=1e-6)     # the map is float32
        f = sum(2.0 ** min(max(float(off[r, 0]) - float(lse[r, 0]), -100), 100) for r in range(t * 128, t * 128 + nrows)) / nrows
        assert math.isclose(se[0, t], f / nrows, rel_tol=1e-9)
        num = sum(float(mass0[0, t, b]) for b in range(nb) if keep[0, t, b]) / nrows
        den = sum(est[b] for b in range(nb) if keep[0, t, b])
        cal = min(max(num / den, 1.0), 64.0) if den > 0 else 1.0
        assert math.isclose(ss[0, t], f * cal, rel_tol=1e-9)


def test_full_step_scales_brute_force():
    L, H = 300, 2
    g = np.random.default_rng(3)
    off = g.normal(5, 1, (384, H)).astype(np.float32)
    lse = off + g.normal(0, 0.3, off.shape).astype(np.float32)
    lse2 = lse.copy()
    se, ss = ref.full_step_scales(off, lse2, L)
    assert (lse2[L:] == 1e30).all() and (ss == 1).all()
    for t in range(3):
        n = min(L - 128 * t, 128)
        for h in range(H):
            f = sum(2.0 ** (float(off[r, h]) - float(lse[r, h])) for r in range(128 * t, 128 * t + n))
            assert math.isclose(se[h, t], f / n / n, rel_tol=1e-9)


# ----------------------------------------------------------------------------------- representatives
def test_block_means_closed_form():
    L, H = 300, 2
    q, k, v = qkv(L, H)
    km, vm = ref.block_means(k, v)
    for b, (r0, r1) in enumerate([(0, 64), (64, 128), (128, 192), (192, 256), (256, 300)]):
        want = torch.from_numpy(k[r0:r1]).double().mean(0).float().to(torch.bfloat16).float().numpy()
        assert np.array_equal(km[b], want)


def test_metric_is_the_query_gram_cholesky():
    L, H, D = 4152, 1, 128
    q, _, _ = qkv(L, H)
    metric, probes = ref.metric_and_probes(q)
    G = q[:, 0].astype(np.float64).T @ q[:, 0] / L / D
    G += 1e-3 * np.mean(np.diag(G)) * np.eye(D)
    M = metric[0].astype(np.float64)
    assert np.allclose(np.triu(M, 1), 0)
    assert np.linalg.norm(M @ M.T - G) / np.linalg.norm(G) < 2e-2          # bf16 factor
    nb = ref.cdiv(L, 64)
    for i in (0, 17, 63):
        blk = int((i * (nb - 1)) / 63 + 0.5)
        r0, r1 = 64 * blk, min(L, 64 * blk + 64)
        assert np.allclose(probes[0, i], q[r0:r1, 0].astype(np.float64).mean(0) / math.sqrt(D), rtol=1e-2,
                           atol=1e-2)


def test_representatives_invariants_and_lloyd_fixed_point():
    L, H, D = 4152, 1, 128
    q, k, v = qkv(L, H, seed=6)
    metric, probes = ref.metric_and_probes(q)
    nb = ref.cdiv(L, 64)
    for j in (0, 10, nb - 1):
        r0, r1 = 64 * j, min(L, 64 * j + 64)
        kk = np.zeros((64, D), np.float32)
        vv = np.zeros((64, D), np.float32)
        kk[:r1 - r0], vv[:r1 - r0] = k[r0:r1, 0], v[r0:r1, 0]
        ck, cv, lc, lab, X, w = ref.kmeans_block(kk, vv, r1 - r0, metric[0], probes[0], iters=100)
        cnt = np.exp2(lc)
        assert math.isclose(cnt.sum(), r1 - r0, rel_tol=1e-12)
        for rep, x in ((ck, kk), (cv, vv)):
            total = (rep.astype(np.float64) * cnt[:, None]).sum(0)
            assert np.linalg.norm(total - x[:r1 - r0].sum(0)) / np.linalg.norm(x[:r1 - r0].sum(0)) < 1e-2
        # converged labels are a fixed point: every valid token is nearest to its own weighted centroid
        valid = np.arange(64) < r1 - r0
        oh = (lab[:, None] == np.arange(4)) & valid[:, None]
        cw = (oh * w[:, None]).sum(0)
        cen = ((oh * w[:, None]).T @ X) / np.maximum(cw, 1e-6)[:, None]
        dist = (cen * cen).sum(1)[None] - 2 * X @ cen.T
        dist = np.where(cw[None] > 0, dist, np.inf)
        assert np.array_equal(np.argmin(dist, 1)[valid], lab[valid])
        assert np.isneginf(lc[cnt == 0]).all() if (cnt == 0).any() else True


def test_kmeans_block_equals_sklearn_weighted_lloyd():
    """The weighted Lloyd loop of kmeans_block against scikit-learn's Lloyd k-means (KMeans(algorithm="lloyd"))
    on the same metric-space points, token weights and starting partition (contiguous quarters of the block):
    converged labels equal, and the representatives are the count-means of those clusters. Probe weights against
    torch.softmax."""
    import torch
    from sklearn.cluster import KMeans
    L, H, D = 4152, 1, 128
    q, k, v = qkv(L, H, seed=8)
    metric, probes = ref.metric_and_probes(q)
    nb = ref.cdiv(L, 64)
    rng = np.random.default_rng(3)
    blocks = [(k[64 * j:64 * j + 64, 0], v[64 * j:64 * j + 64, 0]) for j in list(range(0, nb, 7)) + [nb - 1]]
    # unstructured keys as well: there the clusters move far from the starting quarters
    blocks += [(round_bf16(rng.standard_normal((64 - 5 * (i % 3), D)).astype(np.float32)),
                round_bf16(rng.standard_normal((64 - 5 * (i % 3), D)).astype(np.float32))) for i in range(12)]
    checked = moved = 0
    for kb, vb in blocks:
        n = kb.shape[0]
        kk = np.zeros((64, D), np.float32)
        vv = np.zeros((64, D), np.float32)
        kk[:n], vv[:n] = kb, vb
        ck, cv, lc, lab, X, w = ref.kmeans_block(kk, vv, n, metric[0], probes[0], iters=100)
        sp = torch.as_tensor(probes[0], dtype=torch.float64) @ torch.as_tensor(kk[:n], dtype=torch.float64).T
        w_t = torch.softmax(sp, dim=1).sum(0) * (n / 64)
        assert np.allclose(w[:n], w_t.numpy(), rtol=1e-12, atol=0)
        init_lab = np.arange(n) // 16
        init = np.stack([(w[:n, None] * X[:n])[init_lab == c].sum(0) / w[:n][init_lab == c].sum() for c in range(4)])
        km = KMeans(n_clusters=4, init=init, n_init=1, max_iter=100, tol=0.0, algorithm="lloyd")
        km.fit(X[:n], sample_weight=w[:n])
        if len(np.unique(km.labels_)) < 4:
            continue  # scikit-learn relocates emptied clusters; kmeans_block retires them
        assert np.array_equal(km.labels_, lab[:n])
        moved += int((lab[:n] != init_lab).sum())
        cnt = np.bincount(lab[:n], minlength=4)
        for c in range(4):
            assert lc[c] == np.log2(cnt[c])
            want = ref.round_bf16((kk[:n][lab[:n] == c].astype(np.float64).mean(0)).astype(np.float32))
            assert np.array_equal(ck[c], want)
        checked += 1
    assert checked >= 16 and moved >= 100
