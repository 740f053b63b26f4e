"""numpy restatement of the EchoSparse kernel set -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Every function restates the semantics of one reference kernel (file:line under the reference tree) from its
definition, in float64 for the floating-point work (the "fp32 reference" the GPU result is compared against at
tolerance) and with exact int32 / float32-bit-pattern logic for the plan kernels (compared bit for bit).

Shapes follow the reference: q / k / v are (L, H, D); query tiles have BM = 128 rows (nq = cdiv(L, 128)); kv
blocks have BK = 64 tokens (nb = cdiv(L, 64)); offsets / LSEs are log2 values stored as (nq * 128, H) float32 with
1e30 past L; the block-mass map is (H, nq, nb) float32; block lists are (nq, H, NK) int32; bit plans are
(H, nq, NW) int32 (bit j % 32 of word j // 32 is block j).

Pinning (what checks each function independently of this file; the tests live in tests/test_cpu_oracle.py):
  block_means           closed form; test compares with torch mean + bf16 rounding
  fixed_offset_attention
                        density-1.0 identity with dense softmax attention (torch), offset invariance of O,
                        LSE = prior + log2(sum) identity, brute-force mass map on tiny inputs, check_formula
                        (reference tests/test_attention.py:72-100) re-derived with torch.softmax
  exact_fallback        equals torch.softmax attention over the listed blocks (textbook logsumexp)
  compensate_fallback   closed form: appending mean columns to one softmax (derivation in its docstring),
                        checked against torch.softmax over [exact tokens ++ means]
  estimate_skipped      brute-force per-element loops on tiny inputs
  full_step_scales      brute force on tiny inputs
  select_blocks         hand-made maps with ties, forced and sink blocks, fell-back tiles, NaN (known answers);
                        pack -> rebuild round trip (reference tests/test_sm120.py:109-140)
  pack_plan / rebuild_plan
                        round trip + known answers
  representatives       invariants of reference tests/test_sm120.py:65-83 (weighted sum of reps = block sum,
                        counts sum to block length), Lloyd fixed point, -inf for empty clusters; the weighted
                        Lloyd loop equals scikit-learn's Lloyd k-means on the same points, weights and starting
                        partition, and the probe weights equal torch.softmax (the reference's own clustering
                        uses TF32 dot products, so its float values are matched at tolerance, not bit for bit)
"""
import math

import numpy as np

from .bf16 import round_bf16

BM = 128
BK = 64
LOG2E = 1.4426950408889634
NUM_PROBES = 64


def cdiv(a, b):
    return -(-a // b)


def next_pow2(n):
    return 1 << max(0, (int(n) - 1).bit_length())


def plan_words(nb):
    """Words per (head, tile) of a bit plan (reference echosparse/attention.py:80)."""
    return max(next_pow2(nb) // 32, 4 * cdiv(nb, 128))


def _f64(x):
    return np.asarray(x, dtype=np.float64)


# --------------------------------------------------------------------------------------------- block means
def block_means(k, v):
    """Mean key and value of every 64-token block, (L, H, D) -> (nb, H, D), bf16-rounded (tail block divides by its
    valid token count). Reference: echosparse/kernels/triton_ops.py:21-40."""
    L, H, D = k.shape
    nb = cdiv(L, BK)
    pad = nb * BK - L
    out = []
    for x in (k, v):
        xp = np.concatenate([_f64(x), np.zeros((pad, H, D))], 0).reshape(nb, BK, H, D)
        n = np.minimum(L - np.arange(nb) * BK, BK).astype(np.float64)
        out.append(round_bf16((xp.sum(1) / n[:, None, None]).astype(np.float32)))
    return out[0], out[1]


# --------------------------------------------------------------------------------- fixed-offset attention
def fixed_offset_attention(q, k, v, counts, blocks, offset, threshold=60.0, comp=None, write_mass=False,
                           tiles=None):
    """The fixed-offset pass of one step (reference echosparse/kernels/sm90.py:54-115 with COMP = comp is not None;
    block_attention sm90.py:118-127 is comp=None with the all-blocks list).

    For query tile t and head h, p = 2^(q.k * log2(e)/sqrt(D) - prior[row]) over the keys of the listed exact blocks
    (keys >= L masked), plus (comp) one column per listed mean block (k_mean, v_mean, bias log2(64) or log2(tail)
    for block nb - 1) and four columns per listed refined block (k_rep, v_rep, bias log_counts). total = sum p;
    O = sum p v / total; LSE = prior + log2(total) (1e30 for rows >= L); flag = any valid row with
    |log2 total| > threshold (or NaN); mass[h, t, b] = sum over the tile's valid rows and b's keys of p.

    comp: dict(k_mean, v_mean, means, mean_counts, refine, refine_counts, k_rep, v_rep, log_counts) or None.
    Returns (out (L, H, D) float64, lse (nq*128, H) float64, flags (nq, H) int32, mass (H, nq, nb) or None).
    Rows of tiles >= `tiles` are left as zero / NaN (callers apply launched_tiles semantics)."""
    L, H, D = q.shape
    nq, nb = cdiv(L, BM), cdiv(L, BK)
    tiles = nq if tiles is None else tiles
    scale = LOG2E / math.sqrt(D)
    qf, kf, vf = _f64(q), _f64(k), _f64(v)
    out = np.zeros((L, H, D))
    lse = np.full((nq * BM, H), np.nan)
    flags = np.zeros((nq, H), np.int32)
    mass = np.zeros((H, nq, nb)) if write_mass else None
    tail_log2 = math.log2(L - (nb - 1) * BK)
    for t in range(tiles):
        r0, r1 = t * BM, min(t * BM + BM, L)
        for h in range(H):
            prior = _f64(offset[r0:r1, h])
            qs = qf[r0:r1, h]
            total = np.zeros(r1 - r0)
            acc = np.zeros((r1 - r0, D))
            for b in blocks[t, h, :counts[t, h]]:
                b = int(b)
                c0, c1 = b * BK, min(b * BK + BK, L)
                p = np.exp2(qs @ kf[c0:c1, h].T * scale - prior[:, None])
                total += p.sum(1)
                acc += p @ vf[c0:c1, h]
                if write_mass:
                    mass[h, t, b] = p.sum()
            if comp is not None:
                km, vm = _f64(comp["k_mean"]), _f64(comp["v_mean"])
                ids = np.asarray(comp["means"][t, h, :comp["mean_counts"][t, h]], dtype=np.int64)
                if ids.size:
                    bias = np.where(ids == nb - 1, tail_log2, 6.0)
                    p = np.exp2(qs @ km[ids, h].T * scale + bias[None, :] - prior[:, None])
                    total += p.sum(1)
                    acc += p @ vm[ids, h]
                rids = np.asarray(comp["refine"][t, h, :comp["refine_counts"][t, h]], dtype=np.int64)
                if rids.size:
                    cols = (rids[:, None] * 4 + np.arange(4)[None, :]).reshape(-1)
                    kr, vr = _f64(comp["k_rep"][h, cols]), _f64(comp["v_rep"][h, cols])
                    bias = _f64(comp["log_counts"][h, cols])
                    with np.errstate(invalid="ignore"):
                        p = np.exp2(qs @ kr.T * scale + bias[None, :] - prior[:, None])
                    p = np.where(np.isnan(p), 0.0, p)
                    total += p.sum(1)
                    acc += p @ vr
            with np.errstate(divide="ignore", invalid="ignore"):
                lg = np.log2(total)
                out[r0:r1, h] = acc / total[:, None]
            # a row whose offset is the 1e30 "no row" marker (rows past a tile's valid rows) keeps it, as the
            # kernel keeps 1e30 for rows >= L
            lse[r0:r1, h] = np.where(prior >= 1e30, 1e30, prior + np.where(prior >= 1e30, 0.0, lg))
            lse[r1:t * BM + BM, h] = 1e30
            bad = ~((lg >= -threshold) & (lg <= threshold))
            flags[t, h] = int(bad.any())
    return out, lse, flags, mass


def exact_fallback(q, k, v, out, counts, blocks, lse, flags):
    """Online-softmax attention over the tile's block list for flagged tiles, in place on `out` / `lse` (reference
    echosparse/kernels/sm120.py:143-180; the empty-list convention O = 0, LSE = -1e30 of triton_ops.py:230-234).
    The online recurrence equals the plain softmax, which is what is computed here."""
    L, H, D = q.shape
    nq = cdiv(L, BM)
    scale = LOG2E / math.sqrt(D)
    qf, kf, vf = _f64(q), _f64(k), _f64(v)
    for t in range(nq):
        r0, r1 = t * BM, min(t * BM + BM, L)
        for h in range(H):
            if flags[t, h] == 0:
                continue
            ids = [int(b) for b in blocks[t, h, :counts[t, h]]]
            if not ids:
                out[r0:r1, h] = 0.0
                lse[r0:r1, h] = -1e30
                lse[r1:t * BM + BM, h] = 1e30
                continue
            tok = np.concatenate([np.arange(b * BK, min(b * BK + BK, L)) for b in ids])
            s = qf[r0:r1, h] @ kf[tok, h].T * scale
            m = s.max(1)
            p = np.exp2(s - m[:, None])
            tot = p.sum(1)
            out[r0:r1, h] = p @ vf[tok, h] / tot[:, None]
            lse[r0:r1, h] = m + np.log2(tot)
            lse[r1:t * BM + BM, h] = 1e30


def compensate_fallback(q, k_mean, v_mean, keep, lse, out, flags):
    """Block-mean compensation of the skipped (keep == 0) blocks for flagged tiles, in place (reference
    echosparse/kernels/triton_ops.py:251-295). With e_j = 2^min(q.km_j*s - lse + bias_j, 100):
    O <- (O + sum_j e_j vm_j) / (1 + sum_j e_j), LSE <- LSE + log2(1 + sum_j e_j): appending the mean columns to a
    softmax whose normaliser is 2^LSE."""
    L, H, D = q.shape
    nq, nb = cdiv(L, BM), k_mean.shape[0]
    scale = LOG2E / math.sqrt(D)
    tail_log2 = math.log2(L - (nb - 1) * BK)
    bias = np.full(nb, 6.0)
    bias[nb - 1] = tail_log2
    qf, km, vm = _f64(q), _f64(k_mean), _f64(v_mean)
    for t in range(nq):
        r0, r1 = t * BM, min(t * BM + BM, L)
        for h in range(H):
            if flags[t, h] == 0:
                continue
            sk = keep[h, t] == 0
            l0 = _f64(lse[r0:r1, h])
            e = np.exp2(np.minimum(qf[r0:r1, h] @ km[:, h].T * scale - l0[:, None] + bias[None, :], 100.0))
            e = e * sk[None, :]
            lu = e.sum(1)
            nu = e @ vm[:, h]
            out[r0:r1, h] = (_f64(out[r0:r1, h]) + nu) / (1.0 + lu)[:, None]
            lse[r0:r1, h] = l0 + np.log2(1.0 + lu)
            lse[r1:t * BM + BM, h] = 1e30


# ----------------------------------------------------------------------------------------- map and scales
def estimate_skipped(q, k_mean, keep, offset, lse, mass, NS=16):
    """Mass estimates of skipped blocks and the per-tile scales (reference echosparse/kernels/triton_ops.py:122-177;
    sm120.py:183-250 computes the same values four tiles per program). Writes mass[h, t, b] for keep == 0 blocks in
    place; returns (scale_exact, scale_skip) (H, nq)."""
    L, H, D = q.shape
    nq, nb = cdiv(L, BM), k_mean.shape[0]
    scale = LOG2E / math.sqrt(D)
    lb = np.full(nb, math.log2(BK))
    lb[nb - 1] = math.log2(L - (nb - 1) * BK)
    qf, km = _f64(q), _f64(k_mean)
    se = np.zeros((H, nq))
    ss = np.zeros((H, nq))
    for t in range(nq):
        r = t * BM + np.arange(NS) * (BM // NS)
        rv = r < L
        rr = r[rv]
        nrows = min(L - t * BM, BM)
        rows = np.arange(t * BM, t * BM + nrows)
        for h in range(H):
            ms = _f64(offset[rr, h])
            e = np.exp2(np.minimum(qf[rr, h] @ km[:, h].T * scale - ms[:, None] + lb[None, :], 100.0))
            est = e.sum(0) / max(float(rv.sum()), 1.0)
            ex = keep[h, t] != 0
            num = float(mass[h, t][ex].astype(np.float64).sum())
            den = float(est[ex].sum())
            mass[h, t][~ex] = est[~ex]
            m = _f64(offset[rows, h])
            mn = _f64(lse[rows, h])
            f = np.exp2(np.clip(m - mn, -100.0, 100.0)).sum() / nrows
            se[h, t] = f / nrows
            nn = num / nrows
            c = min(max(nn / max(den, 1e-30), 1.0), 64.0) if den > 0 else 1.0
            ss[h, t] = f * c
    return se, ss


def full_step_scales(offset, lse, L):
    """Scales after a step that computed every block; resets lse rows >= L to 1e30 in place (reference
    echosparse/kernels/triton_ops.py:180-199). Returns (scale_exact, scale_skip) (H, nq)."""
    nqbm, H = offset.shape
    nq = nqbm // BM
    se = np.zeros((H, nq))
    ss = np.ones((H, nq))
    lse[L:] = 1e30
    for t in range(nq):
        nrows = min(L - t * BM, BM)
        rows = np.arange(t * BM, t * BM + nrows)
        for h in range(H):
            f = np.exp2(np.clip(_f64(offset[rows, h]) - _f64(lse[rows, h]), -100.0, 100.0))
            se[h, t] = f.sum() / nrows / nrows
    return se, ss


# -------------------------------------------------------------------------------- selection and the plans
def _bits(x):
    return np.asarray(x, dtype=np.float32).view(np.int32)


def kth_largest_bits(bits, K):
    """The value the reference's 31-step bisection returns (echosparse/kernels/triton_ops.py:43-54): the largest
    int32 x in [0, 0x7F800001) with count(bits >= x) >= K, i.e. the K-th largest bit pattern when at least K
    patterns are >= 0, else 0 (and 0x7F800000 when K <= 0)."""
    bits = np.asarray(bits, dtype=np.int64)
    if K <= 0:
        return 0x7F800000
    nonneg = np.sort(bits[bits >= 0])[::-1]
    if nonneg.size < K:
        return 0
    return int(min(nonneg[K - 1], 0x7F800000))


def select_blocks(mass, keep_prev, scale_exact, scale_skip, flags, k, r, L, refine_width, words, sink=1 << 30):
    """Top-k blocks of every (tile, head) plus forced ones, the refine list and the skip bit mask (reference
    echosparse/kernels/triton_ops.py:57-119). All float work is float32 elementwise (one multiply), exactly as the
    kernel does it. Returns keep (H,nq,nb) u8, counts (nq,H), blocks (nq,H,nb) (entries past the count are 0),
    refine (nq,H,RW) padded with nb, skip (H,nq,words) int32 (words past next_pow2(nb)/32 are -1)."""
    H, nq, nb = mass.shape
    nbp = max(32, next_pow2(nb))       # (the reference needs nb >= 32; shorter maps use one word)
    keep = np.zeros((H, nq, nb), np.uint8)
    counts = np.zeros((nq, H), np.int32)
    blocks = np.zeros((nq, H, nb), np.int32)
    refine = np.full((nq, H, refine_width), nb, np.int32)
    skip = np.full((H, nq, words), -1, np.int32)
    j = np.arange(nb)
    for t in range(nq):
        lo = (t * BM) // BK - 1
        hi = (min((t + 1) * BM, L) - 1) // BK + 1
        forced = ((j >= lo) & (j <= hi)) | (j >= sink)
        for h in range(H):
            kept_before = keep_prev[h, t] != 0
            raw = np.asarray(mass[h, t], np.float32)
            se = np.float32(scale_exact[h, t])
            ss = np.float32(scale_skip[h, t])
            with np.errstate(invalid="ignore", over="ignore"):
                val = np.where(kept_before, np.where(flags[t, h] != 0, np.float32(np.inf), raw * se), raw * ss)
            val = np.where(np.isnan(val), np.float32(0.0), val).astype(np.float32)
            val = np.where(j >= sink, np.float32(np.inf), val).astype(np.float32)
            thr_bits = kth_largest_bits(_bits(val), k)
            thr = np.array([thr_bits], np.int32).view(np.float32)[0]
            kp = (val >= thr) | forced
            r2 = np.where(np.isnan(raw), np.float32(0.0), raw).astype(np.float32)
            r2 = np.where(~kp, r2, np.float32(-1.0)).astype(np.float32)
            rb = _bits(r2)
            ref = (rb >= kth_largest_bits(rb, int(r))) & (r2 >= 0.0) if r > 0 else np.zeros(nb, bool)
            ref &= (np.cumsum(ref) - 1) < r
            nref = int(ref.sum())
            refine[t, h, :] = nb
            refine[t, h, :nref] = j[ref][:refine_width]
            keep[h, t] = kp
            idx = j[kp]
            counts[t, h] = idx.size
            blocks[t, h, :idx.size] = idx
            sk = np.ones(nbp, bool)
            sk[:nb] = kp | ref
            skip[h, t, :nbp // 32] = _pack_words(sk)
    return keep, counts, blocks, refine, skip


def _pack_words(bits):
    """bool array of length 32*n -> n int32 words, bit i of word w = bits[32*w + i]."""
    b = np.asarray(bits, bool).reshape(-1, 32).astype(np.uint64)
    w = (b << np.arange(32, dtype=np.uint64)[None, :]).sum(1)
    return w.astype(np.uint32).view(np.int32)


def _unpack_words(words, n):
    w = np.asarray(words, np.int32).view(np.uint32).astype(np.uint64)
    b = (w[..., :, None] >> np.arange(32, dtype=np.uint64)) & 1
    return b.reshape(*w.shape[:-1], -1)[..., :n].astype(bool)


def pack_plan(keep, words):
    """keep (H, nq, nb) -> exact bit mask (H, nq, words) int32, bit set also for j >= nb (reference
    echosparse/kernels/sm120.py:258-273). Words past next_pow2(nb)/32 are not written by the reference; they are
    -1 here (the plans' initial value)."""
    H, nq, nb = keep.shape
    nbp = max(32, next_pow2(nb))
    out = np.full((H, nq, words), -1, np.int32)
    for h in range(H):
        for t in range(nq):
            b = np.ones(nbp, bool)
            b[:nb] = keep[h, t] != 0
            out[h, t, :nbp // 32] = _pack_words(b)
    return out


def rebuild_plan(exact_bits, skip_bits, nb, refine_width):
    """Bit plans -> keep (H,nq,nb) u8, counts (nq,H), blocks (nq,H,nb), refine (nq,H,RW) padded with nb,
    refine_counts (nq,H), means (nq,H,nb), mean_counts (nq,H) (reference echosparse/kernels/sm120.py:276-305).
    List entries past the counts are left 0."""
    H, nq, _ = exact_bits.shape
    ex = _unpack_words(exact_bits, nb)
    sk = _unpack_words(skip_bits, nb)
    keep = ex.astype(np.uint8)
    counts = np.zeros((nq, H), np.int32)
    blocks = np.zeros((nq, H, nb), np.int32)
    refine = np.full((nq, H, refine_width), nb, np.int32)
    rcounts = np.zeros((nq, H), np.int32)
    means = np.zeros((nq, H, nb), np.int32)
    mcounts = np.zeros((nq, H), np.int32)
    j = np.arange(nb)
    for h in range(H):
        for t in range(nq):
            e, s = ex[h, t], sk[h, t]
            ids = j[e]
            counts[t, h] = ids.size
            blocks[t, h, :ids.size] = ids
            m = j[~s]
            mcounts[t, h] = m.size
            means[t, h, :m.size] = m
            rf = j[s & ~e]
            n = min(rf.size, refine_width)
            refine[t, h, :n] = rf[:n]
            rcounts[t, h] = n
    return keep, counts, blocks, refine, rcounts, means, mcounts


def budget(density, nb):
    """Exact blocks and refined blocks per tile (reference echosparse/attention.py:267-270)."""
    top = max(1, int(round(density * nb)))
    return top, max(0, int(round((nb - top) / 3)))


# ------------------------------------------------------------------------------------------ representatives
def metric_and_probes(q):
    """Query-metric Cholesky factor (H, D, D) and 64 probe queries (H, 64, D), both bf16-rounded (reference
    echosparse/kernels/representatives.py:22-63,156-166): G = E[q q^T] * scale^2 + 1e-3 * mean(diag) * I,
    lower Cholesky factor with pivots clamped at mean(diag) * 1e-12; probe i = scale * mean of the valid q rows of
    block round(i * (nb - 1) / 63)."""
    L, H, D = q.shape
    nb = cdiv(L, BK)
    scale = D ** -0.5
    qf = _f64(q)
    metric = np.zeros((H, D, D), np.float32)
    probes = np.zeros((H, NUM_PROBES, D), np.float32)
    for h in range(H):
        g = qf[:, h].T @ qf[:, h] * (scale * scale / L)
        g = g + 1e-3 * np.mean(np.diag(g)) * np.eye(D)
        metric[h] = round_bf16(_cholesky_clamped(g).astype(np.float32))
        for i in range(NUM_PROBES):
            blk = int(np.float32(i * (nb - 1)) / np.float32(NUM_PROBES - 1) + np.float32(0.5))
            r0, r1 = blk * BK, min(blk * BK + BK, L)
            probes[h, i] = round_bf16((qf[r0:r1, h].sum(0) * scale / max(r1 - r0, 1)).astype(np.float32))
    return metric, probes


def _cholesky_clamped(A):
    """Right-looking lower Cholesky with the reference's pivot clamp (representatives.py:49-63)."""
    A = np.array(A, np.float64)
    D = A.shape[0]
    eps = np.trace(A) / D * 1e-12
    Lm = np.zeros_like(A)
    for j in range(D):
        piv = max(A[j, j], eps)
        col = np.where(np.arange(D) >= j, A[:, j] / math.sqrt(piv), 0.0)
        Lm[:, j] = col
        A -= np.outer(col, col)
    return Lm


def kmeans_block(kk, vv, nvalid, metric, probes, iters):
    """Weighted Lloyd of one block's keys in the query metric (reference representatives.py:66-128). kk, vv: (64, D)
    bf16 values (rows >= nvalid are zero). Returns (k_rep (4, D), v_rep (4, D), log2 counts (4,), labels (64,),
    X (64, D), weights (64,))."""
    tok = np.arange(BK)
    valid = tok < nvalid
    X = _f64(kk) @ _f64(metric)
    sp = _f64(probes) @ _f64(kk).T
    sp = np.where(valid[None, :], sp, -np.inf)
    e = np.exp(sp - sp.max(1, keepdims=True))
    e = e / e.sum(1, keepdims=True)
    w = np.where(valid, e.sum(0) * (valid.sum() / NUM_PROBES), 0.0)
    lab = tok // (BK // 4)

    def centroids(lab):
        oh = (lab[:, None] == np.arange(4)[None, :]) & valid[:, None]
        ohw = oh * w[:, None]
        cw = ohw.sum(0)
        return oh, cw, (ohw.T @ X) / np.maximum(cw, 1e-6)[:, None]

    oh, cw, cen = centroids(lab)
    it, changed = 0, 1
    while it < iters and changed > 0:
        dist = (cen * cen).sum(1)[None, :] - 2.0 * X @ cen.T
        dist = np.where((cw > 0)[None, :], dist, np.inf)
        new = np.argmin(dist, 1)
        changed = int(((new != lab) & valid).sum())
        lab = new
        oh, cw2, cen2 = centroids(lab)
        cen = np.where((cw2 > 0)[:, None], cen2, cen)
        cw = cw2
        it += 1
    cnt = oh.sum(0).astype(np.float64)
    inv = 1.0 / np.maximum(cnt, 1.0)
    ck = round_bf16(((oh.T.astype(np.float64) @ _f64(kk)) * inv[:, None]).astype(np.float32))
    cv = round_bf16(((oh.T.astype(np.float64) @ _f64(vv)) * inv[:, None]).astype(np.float32))
    with np.errstate(divide="ignore"):
        lc = np.where(cnt > 0, np.log2(np.maximum(cnt, 1.0)), -np.inf)
    return ck, cv, lc, lab, X, w


def representatives(q, k, v, iters=6):
    """Four representatives per block: (k_rep, v_rep) (H, (nb+1)*4, D) and log_counts (H, (nb+1)*4); block nb is
    the empty sentinel (zeros, -inf). Reference echosparse/kernels/representatives.py:131-166."""
    L, H, D = q.shape
    nb = cdiv(L, BK)
    metric, probes = metric_and_probes(q)
    kr = np.zeros((H, (nb + 1) * 4, D), np.float32)
    vr = np.zeros_like(kr)
    lc = np.full((H, (nb + 1) * 4), -np.inf, np.float32)
    for h in range(H):
        for j in range(nb):
            r0, r1 = j * BK, min(j * BK + BK, L)
            kk = np.zeros((BK, D), np.float32)
            vv = np.zeros((BK, D), np.float32)
            kk[:r1 - r0] = k[r0:r1, h]
            vv[:r1 - r0] = v[r0:r1, h]
            ck, cv, c, *_ = kmeans_block(kk, vv, r1 - r0, metric[h], probes[h], iters)
            kr[h, 4 * j:4 * j + 4], vr[h, 4 * j:4 * j + 4], lc[h, 4 * j:4 * j + 4] = ck, cv, c
    return kr, vr, lc
