"""numpy restatement of the VSA / VSA2 path -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Tokens are [B, H, L, D] with L = NB * 64 and blk_cnt [NB] valid tokens per block (valid-first); selections are
bool block masks [B, H, NB, NB] or CSR (ptr [B, H, NB + 1], idx). Floating-point work is float64 unless a function
restates a kernel's float32 / bf16 arithmetic order on purpose (then it says so and is compared bit for bit).

Functions and what pins each one (tests/test_cpu_vsa_oracle.py):
  token_valid, pool        pool restates pool.cu's float32 order (rows of a group in order, then the groups; times
                           the reciprocal count, bf16 round): pinned against float64 means within fp32 rounding and
                           by padding never being read (NaN padding keeps outputs finite)
  block_scores             rnd(rnd(qc . kc) / sqrt(D)) from given means (reference tests/vsa_reference.py:148-151):
                           float64 dot, so it pins the GPU value up to one bf16 step of the dot's rounding
  row_topk_mask            known-answer vector of reference tests/test_vsa.py:67-73 (ties, -0 == +0, K bounds)
                           and brute force over Python's stable sort
  global_topk_mask         exact count per (b, h), brute-force flat order (reference tests/vsa_reference.py:77-87)
  psp_scores               rows sum to 1 under valid_groups with every group valid (reference
                           tests/test_vsa2.py:169-170), paper = valid_groups / G for full blocks, and a brute-force
                           per-element loop on a tiny case
  fine_attention           full mask == dense softmax attention (torch scaled_dot_product_attention, float64), empty
                           rows -> O = 0 / lse = -inf, permutation of the kv blocks leaves O unchanged
  fine_backward            analytic gradients, pinned against torch.autograd on the float64 forward
  fuse_fwd / fuse_bwd      torch.autograd of the fusion formula (reference csrc/vsa/fuse.cu:3-9)
  vsa_output               the full operator for a frozen mask (reference tests/vsa_reference.py:110-135) in torch
                           float64 with autograd; pinned by the fine / coarse pieces above and by the identity that
                           the empty mask leaves only the coarse branch (reference tests/test_vsa.py:76-84)
  plan_reference           the split planner's contract (reference tests/test_vsa2_split.py:60-87), pinned by hand
                           cases and by every edge being covered exactly once
  merge_fwd                LSE merge of normalized partials equals the unsplit softmax (closed form)
  kmeans_seed_tokens       distinct in-range tokens, deterministic per (seed, bh, blk), varying with the seed
  kmeans_tables            counts partition the valid tokens, rows are the float64 means of their members, empty
                           clusters retire; centroids equal scikit-learn's Lloyd k-means started from the same seed
                           tokens for the same number of rounds
  row_tiers                exact per-row counts, A inside A|B, brute-force order with ties and -0 / +0
  rep_fine_head            blockwise analytic forward / backward of one head: equals rep_fine_torch and its
                           autograd gradients (contiguous and k-means groups, empty groups, empty rows)
  rep_kv_block_grads       one kv block's dK / dV from the backward's inputs: equals rep_fine_head's rows
"""
import math

import numpy as np

from .bf16 import round_bf16

BLOCK = 64


def token_valid(blk_cnt, L):
    """bool [L]: position p is valid iff p % 64 < blk_cnt[p // 64] (reference tests/vsa_reference.py:27-29)."""
    pos = np.arange(L)
    return (pos % BLOCK) < np.asarray(blk_cnt, np.int64)[pos // BLOCK]


def pool(x, blk_cnt, R, rnd=round_bf16):
    """(group means [B, H, NB * G, D], block means [B, H, NB, D]) as 16-bit values in float32 (rnd: round_bf16 or
    round_f16, the token dtype), restating csrc/vsa/router/pool.cu:16-51: per column, float32 sums of a group's
    valid rows in order, the group sums added in order, times 1 / count; empty groups give 0."""
    x = np.asarray(x, np.float32)
    B, H, L, D = x.shape
    NB, G = L // BLOCK, BLOCK // R
    cnt = np.asarray(blk_cnt, np.int64)
    grp = np.zeros((B, H, NB * G, D), np.float32)
    blk = np.zeros((B, H, NB, D), np.float32)
    for b in range(NB):
        tot = np.zeros((B, H, D), np.float32)
        for g in range(G):
            r0, r1 = g * R, min(g * R + R, int(cnt[b]))
            s = np.zeros((B, H, D), np.float32)
            for r in range(r0, r1):
                s = (s + x[:, :, b * BLOCK + r]).astype(np.float32)
            inv = np.float32(1.0) / np.float32(r1 - r0) if r1 > r0 else np.float32(0.0)
            grp[:, :, b * G + g] = rnd(s * inv)
            tot = (tot + s).astype(np.float32)
        blk[:, :, b] = rnd(tot * (np.float32(1.0) / np.float32(cnt[b])))
    return grp, blk


def block_scores(qc, kc, rnd=round_bf16):
    """rnd(rnd(qc . kc) / sqrt(D)) with rnd the token dtype's rounding (bf16 default), float64 dot (reference
    tests/vsa_reference.py:148-151)."""
    qc, kc = np.asarray(qc, np.float64), np.asarray(kc, np.float64)
    D = qc.shape[-1]
    s = rnd(np.einsum("...id,...jd->...ij", qc, kc).astype(np.float32))
    return rnd((s * np.float32(1.0 / math.sqrt(D))).astype(np.float32))


def _desc_order(values):
    """Indices sorting a 1-D float array by value descending, ties by smaller index (-0 == +0)."""
    v = np.asarray(values, np.float64) + 0.0
    return np.lexsort((np.arange(v.size), -v))


def row_topk_mask(scores, K):
    """Exactly min(K, NB) blocks per row, score desc, ties to the smaller index (reference
    tests/vsa_reference.py:160-165)."""
    s = np.asarray(scores, np.float64)
    k = max(0, min(int(K), s.shape[-1]))
    flat = s.reshape(-1, s.shape[-1])
    mask = np.zeros(flat.shape, bool)
    for r in range(flat.shape[0]):
        mask[r, _desc_order(flat[r])[:k]] = True
    return mask.reshape(s.shape)


def global_topk_mask(scores, budget):
    """Exactly min(budget, NB^2) entries per (b, h), score desc then flat index asc (reference
    tests/vsa_reference.py:77-87)."""
    s = np.asarray(scores, np.float64)
    B, H, NB, _ = s.shape
    k = max(0, min(int(budget), NB * NB))
    flat = s.reshape(B * H, NB * NB)
    mask = np.zeros(flat.shape, bool)
    for r in range(flat.shape[0]):
        mask[r, _desc_order(flat[r])[:k]] = True
    return mask.reshape(s.shape)


def group_valid(blk_cnt, R):
    """bool [NB * G]: a pooled group is valid iff it holds >= 1 valid token."""
    cnt = np.asarray(blk_cnt, np.int64)
    G = BLOCK // R
    g = np.arange(cnt.size * G)
    return (g % G) * R < cnt[g // G]


def psp_scores(qr, kr, blk_cnt, R, row_norm):
    """VSA2 PSP block scores [B, H, NB, NB] from given pooled rows qr / kr [B, H, >= NB * G, D] (float64):
    A = softmax over all valid pooled keys of qr . kr / sqrt(D), zero rows for invalid pooled queries, summed over
    (query group in i, key group in j), times 1 / G^2 (row_norm 1, "paper") or 1 / #valid groups of i (row_norm 0)
    (reference csrc/vsa/router/router.cu:1-15, tests/vsa_reference.py:56-74)."""
    cnt = np.asarray(blk_cnt, np.int64)
    NB, G = cnt.size, BLOCK // R
    Lr = NB * G
    q = np.asarray(qr, np.float64)[:, :, :Lr]
    k = np.asarray(kr, np.float64)[:, :, :Lr]
    D = q.shape[-1]
    gv = group_valid(cnt, R)
    s = np.einsum("bhid,bhjd->bhij", q, k) / math.sqrt(D)
    s = np.where(gv[None, None, None, :], s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    a = np.exp(s)
    a = a / a.sum(-1, keepdims=True) * gv[None, None, :, None]
    B, H = q.shape[:2]
    S = a.reshape(B, H, NB, G, NB, G).sum((3, 5))
    if row_norm == 1:
        return S / (G * G)
    return S / ((cnt + R - 1) // R)[None, None, :, None]


def csr_from_mask(mask):
    """(ptr [B, H, NB + 1] int32 absolute, idx int32) of a bool mask [B, H, NB, NB], rows ascending."""
    m = np.asarray(mask, bool)
    B, H, N, _ = m.shape
    rows = m.reshape(-1, N)
    ends = np.cumsum(rows.sum(1))
    starts = ends - rows.sum(1)
    ptr = np.concatenate([starts.reshape(B * H, N), ends.reshape(B * H, N)[:, -1:]], 1).reshape(B, H, N + 1)
    idx = np.nonzero(rows)[1]
    return ptr.astype(np.int32), idx.astype(np.int32)


def mask_from_csr(ptr, idx, nb):
    ptr, idx = np.asarray(ptr, np.int64), np.asarray(idx, np.int64)
    B, H = ptr.shape[:2]
    m = np.zeros((B, H, nb, nb), bool)
    for b in range(B):
        for h in range(H):
            for i in range(nb):
                m[b, h, i, idx[ptr[b, h, i]:ptr[b, h, i + 1]]] = True
    return m


def fine_attention(q, k, v, blk_cnt, mask):
    """(O [B, H, L, D], lse [B, H, L] natural) of attention restricted to the selected blocks with invalid keys
    masked; rows with nothing to attend and padding rows give O = 0, lse = -inf (reference
    tests/vsa_reference.py:90-107, csrc/vsa/generic/attn_fwd.cu:16-24). float64."""
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    B, H, L, D = q.shape
    valid = token_valid(blk_cnt, L)
    blk = np.arange(L) // BLOCK
    allowed = np.asarray(mask, bool)[:, :, blk][:, :, :, blk] & valid[None, None, None, :]
    s = np.einsum("bhid,bhjd->bhij", q, k) / math.sqrt(D)
    s = np.where(allowed, s, -np.inf)
    has = allowed.any(-1) & valid[None, None, :]
    m = np.where(has, s.max(-1), 0.0)
    p = np.where(allowed, np.exp(s - m[..., None]), 0.0)
    l = p.sum(-1)
    o = np.einsum("bhij,bhjd->bhid", p / np.where(has, l, 1.0)[..., None], v) * has[..., None]
    lse = np.where(has, m + np.log(np.where(has, l, 1.0)), -np.inf)
    return o, lse


def fine_backward(q, k, v, blk_cnt, mask, dout):
    """(dq, dk, dv) of fine_attention for upstream dO, float64 closed form: P = softmax, dV = P^T dO,
    dP = dO V^T, dS = P (dP - rowsum(dO * O)), dQ = dS K / sqrt(D), dK = dS^T Q / sqrt(D); padding rows of dO are
    ignored (their P is 0)."""
    q, k, v, dout = (np.asarray(x, np.float64) for x in (q, k, v, dout))
    B, H, L, D = q.shape
    o, lse = fine_attention(q, k, v, blk_cnt, mask)
    valid = token_valid(blk_cnt, L)
    blk = np.arange(L) // BLOCK
    allowed = np.asarray(mask, bool)[:, :, blk][:, :, :, blk] & valid[None, None, None, :] & valid[None, None, :, None]
    s = np.einsum("bhid,bhjd->bhij", q, k) / math.sqrt(D)
    p = np.where(allowed, np.exp(s - np.where(np.isfinite(lse), lse, 0.0)[..., None]), 0.0)
    delta = (dout * o).sum(-1)
    dv = np.einsum("bhij,bhid->bhjd", p, dout)
    dp = np.einsum("bhid,bhjd->bhij", dout, v)
    ds = p * (dp - delta[..., None])
    dq = np.einsum("bhij,bhjd->bhid", ds, k) / math.sqrt(D)
    dk = np.einsum("bhij,bhid->bhjd", ds, q) / math.sqrt(D)
    keep = valid[None, None, :, None]
    return dq * keep, dk * keep, dv * keep


def vsa_output(q, k, v, gate, blk_cnt, mask, gate_act="tanh", pooled=None):
    """The full operator for a frozen mask as a torch float64 graph (autograd gives the gradients):
    O = (O_fine + act(gate) * O_coarse[blk]) on valid rows, 0 elsewhere, O_coarse = softmax(qc kc^T / sqrt(D)) vc
    over the block means (reference tests/vsa_reference.py:110-135, csrc/vsa/fuse.cu:3). q / k / v / gate are torch
    float64 tensors; `pooled` optionally overrides (qc, kc, vc) values (e.g. the bf16-rounded means the kernels
    use) while keeping the mean's gradient path (straight-through)."""
    import torch
    B, H, L, D = q.shape
    NB = L // BLOCK
    valid = torch.as_tensor(token_valid(blk_cnt, L))
    cnt = torch.as_tensor(np.asarray(blk_cnt, np.float64))
    z = valid[None, None, :, None].to(q.dtype)

    def mean(x):
        return (x * z).reshape(B, H, NB, BLOCK, D).sum(3) / cnt[None, None, :, None]

    qc, kc, vc = mean(q), mean(k), mean(v)
    if pooled is not None:
        qc, kc, vc = (m + (torch.as_tensor(np.asarray(p, np.float64)) - m).detach() for m, p in zip((qc, kc, vc), pooled))
    oc = torch.softmax(qc @ kc.transpose(-1, -2) / math.sqrt(D), -1) @ vc
    blk = torch.arange(L) // BLOCK
    allowed = torch.as_tensor(np.asarray(mask, bool))[:, :, blk][:, :, :, blk] & valid[None, None, None, :]
    s = (q @ k.transpose(-1, -2)) / math.sqrt(D)
    s = s.masked_fill(~allowed, float("-inf"))
    has = allowed.any(-1, keepdim=True)
    p = torch.softmax(torch.where(has, s, torch.zeros_like(s)), -1) * has
    of = p @ v
    if gate is None:
        a = torch.ones_like(of[..., :1])
    else:
        a = torch.tanh(gate) if gate_act == "tanh" else gate
        if gate.dim() == 3:
            a = a[..., None]
    return (of + a * oc[:, :, blk]) * z


def plan_reference(ptr, chunk, max_slots, min_len=0, rel_mean=0.0, tail_frac=0.0, resident=1, budget=-1):
    """The split-KV planner's contract in plain Python: (tasks, merges, info[8]) (reference
    tests/test_vsa2_split.py:60-87, csrc/vsa/split.cu:1-19)."""
    p = np.asarray(ptr, np.int64)
    B, H, n1 = p.shape
    nb = n1 - 1
    rows_ptr = p.reshape(B * H, n1)
    W = int(rows_ptr[-1, -1] - rows_ptr[0, 0])
    gthr = max(chunk + 1, min_len)
    if tail_frac > 0:
        gthr = max(gthr, math.ceil(tail_frac * W / resident))
    cap = 2 ** 31 - 1 if budget < 0 else budget
    rows = []
    for bh in range(B * H):
        hp = rows_ptr[bh]
        thr = gthr if rel_mean <= 0 else max(gthr, math.ceil(rel_mean * int(hp[nb] - hp[0]) / nb))
        for i in range(nb):
            n = int(hp[i + 1] - hp[i])
            rows.append((bh * nb + i, int(hp[i]), n, n >= thr))
    E = sum(1 for r in rows if r[3])
    ok = E <= cap
    split, direct, merges, used = [], [], [], 0
    for r, beg, n, elig in rows:
        c = -(-n // chunk) if elig else 0
        if ok and c and used + c <= max_slots:
            merges.append([r, used, c, 0])
            split += [[r, beg + j * n // c, beg + (j + 1) * n // c, used + j] for j in range(c)]
        else:
            direct.append([r, beg, beg + n, -1])
        used += c
    t_split = sum(m[2] for m in merges)
    info = [len(split) + len(direct), len(merges), t_split, len(rows), E, int(ok), gthr, W]
    return split + direct, merges, info


def merge_fwd(part_o, part_lse2):
    """(o, lse natural) of normalized partials with log2 LSEs: weights 2^(lse_i - M) (reference
    csrc/vsa/split.cu:16-19)."""
    po, pl = np.asarray(part_o, np.float64), np.asarray(part_lse2, np.float64)
    M = pl.max(0)
    w = np.exp2(pl - np.where(np.isfinite(M), M, 0.0))
    w = np.where(np.isfinite(pl), w, 0.0)
    s = w.sum(0)
    o = (w[..., None] * po).sum(0) / np.where(s > 0, s, 1.0)[..., None]
    lse = np.where(s > 0, (M + np.log2(np.where(s > 0, s, 1.0))) * math.log(2.0), -np.inf)
    return o, lse


# --------------------------------------------------------------------------- VSA2 three-tier representatives
def rep_tables(k, v, blk_cnt, RM, rnd=round_bf16):
    """(k_mid, v_mid [B, H, NB * RM, D], k_tail, v_tail [B, H, NB, D], lc_mid [NB * RM], lc_tail [NB]): the pooled
    group / block means of the kernels' float32 order (see `pool`, groups of 64 / RM tokens) and log2 counts, -inf
    for an empty group (reference experiments/vsa2_representative/vsa2_rep/reference.py:23-50); rnd = the token
    dtype's rounding."""
    km, kt = pool(k, blk_cnt, BLOCK // RM, rnd)
    vm, vt = pool(v, blk_cnt, BLOCK // RM, rnd)
    cnt = np.asarray(blk_cnt, np.int64)
    gs = BLOCK // RM
    n = np.clip(cnt[:, None] - np.arange(RM)[None, :] * gs, 0, gs).reshape(-1)
    with np.errstate(divide="ignore"):
        lc_mid = np.where(n > 0, np.log2(np.maximum(n, 1)), -np.inf)
        lc_tail = np.log2(cnt.astype(np.float64))
    return km, vm, kt, vt, lc_mid, lc_tail


def rep_fine_torch(q, k, v, blk_cnt, mask_a, mask_ab, RM, phases=7, tables=None, labels=None):
    """Three-tier attention as a torch float64 graph: one softmax over tier-A tokens (mask_a), tier-B representatives
    (mask_ab & ~mask_a; means of 64 / RM-token groups with + ln c) and tier-C block means (~mask_ab, + ln cnt); O = 0
    and lse = -inf on padding rows and rows with no column (reference vsa2_rep/reference.py:53-96). The means are
    functions of k / v (so autograd reaches the tokens); `tables` = (k_mid, v_mid, k_tail, v_tail) overrides their
    values (e.g. the bf16 tables the kernels use) straight-through. `labels` [B, H, L] (-1 on padding) replaces the
    contiguous groups by clusters: representative c of a block is the mean of its tokens labelled c (k-means
    tables). Returns (O, lse natural)."""
    import torch
    B, H, L, D = q.shape
    NB, gs = L // BLOCK, BLOCK // RM
    cnt = np.asarray(blk_cnt, np.int64)
    valid = torch.as_tensor(token_valid(cnt, L))
    z = valid[None, None, :, None].to(q.dtype)
    blk = np.arange(L) // BLOCK
    if labels is None:
        grp = np.where(token_valid(cnt, L), blk * RM + (np.arange(L) % BLOCK) // gs, -1)
        grp = np.broadcast_to(grp, (B, H, L))
    else:
        lab = np.asarray(labels, np.int64)
        grp = np.where(lab >= 0, blk[None, None, :] * RM + lab, -1)
    member = torch.as_tensor(grp[..., None, :] == np.arange(NB * RM)[:, None]).to(q.dtype)   # [B, H, NB*RM, L]
    ng = member.sum(-1)                                                                        # [B, H, NB*RM]

    def means(x):
        xs = member @ (x * z)
        mid = xs / ng.clamp(min=1)[..., None]
        tail = xs.reshape(B, H, NB, RM, D).sum(3) / torch.as_tensor(cnt, dtype=q.dtype)[None, None, :, None]
        return mid, tail

    km, kt = means(k)
    vm, vt = means(v)
    if tables is not None:
        over = [torch.as_tensor(np.asarray(t, np.float64)) for t in tables]
        km, vm, kt, vt = (m + (o - m).detach() for m, o in zip((km, vm, kt, vt), over))
    a = np.asarray(mask_a, bool) & bool(phases & 1)
    ab = np.asarray(mask_ab, bool)
    tb = (ab & ~np.asarray(mask_a, bool)) & bool(phases & 2)
    tc = (~ab) & bool(phases & 4)
    blk = np.arange(L) // BLOCK
    vis_a = a[:, :, blk][:, :, :, blk] & token_valid(cnt, L)[None, None, None, :]
    vis_b = np.repeat(tb, RM, axis=3)[:, :, blk] & (ng.numpy() > 0)[:, :, None, :]
    vis_c = tc[:, :, blk]
    vis = torch.as_tensor(np.concatenate([vis_a, vis_b, vis_c], axis=3))
    with np.errstate(divide="ignore"):
        bias = np.concatenate([np.zeros((B, H, L)), np.log(np.maximum(ng.numpy(), 1)),
                               np.broadcast_to(np.log(cnt), (B, H, NB))], axis=2)
        bias = torch.as_tensor(bias)[:, :, None, :]
    Kc = torch.cat([k, km, kt], 2)
    Vc = torch.cat([v, vm, vt], 2)
    s = (q @ Kc.transpose(-1, -2)) / math.sqrt(D) + bias
    s = s.masked_fill(~vis, float("-inf"))
    has = vis.any(-1, keepdim=True) & valid[None, None, :, None]
    s_safe = torch.where(has, s, torch.zeros_like(s))
    p = torch.softmax(s_safe, -1) * has
    o = p @ Vc
    lse = torch.where(has[..., 0], torch.logsumexp(s_safe, -1), torch.full_like(s[..., 0], float("-inf")))
    return o, lse


def fine_attention_blocks(q, k, v, blk_cnt, ptr, idx, bh, qblocks):
    """Blockwise float32 CPU port of the fine forward over CSR lists for the listed query blocks of head bh only:
    (O [n, 64, D], lse [n, 64]); never materialises L x L (the CPU-baseline leg of bench.py times this). Pinned by
    agreeing with fine_attention on the same inputs (tests/test_cpu_vsa_oracle.py)."""
    q, k, v = (np.asarray(x[bh], np.float32) for x in (q, k, v))
    D = q.shape[-1]
    cnt = np.asarray(blk_cnt, np.int64)
    p = np.asarray(ptr, np.int64).reshape(-1, cnt.size + 1)[bh]
    cols = np.asarray(idx, np.int64)
    outs, lses = [], []
    for i in qblocks:
        qs = q[i * BLOCK:(i + 1) * BLOCK] * np.float32(1.0 / math.sqrt(D))
        blocks = cols[p[i]:p[i + 1]]
        m = np.full(BLOCK, -np.inf, np.float32)
        l = np.zeros(BLOCK, np.float32)
        o = np.zeros((BLOCK, D), np.float32)
        for j in blocks:
            n = int(cnt[j])
            s = qs @ k[j * BLOCK:j * BLOCK + n].T
            mn = np.maximum(m, s.max(1))
            a = np.exp(m - mn)
            e = np.exp(s - mn[:, None])
            l = l * a + e.sum(1)
            o = o * a[:, None] + e @ v[j * BLOCK:j * BLOCK + n]
            m = mn
        live = (l > 0) & (np.arange(BLOCK) < cnt[i])
        outs.append(np.where(live[:, None], o / np.where(live, l, 1)[:, None], 0))
        lses.append(np.where(live, m + np.log(np.where(live, l, 1)), -np.inf))
    return np.stack(outs), np.stack(lses)


def rep_fine_head(q, k, v, blk_cnt, mask_a, mask_ab, RM, tables, groups, dout, o_delta=None):
    """Blockwise float64 three-tier attention of ONE head with analytic gradients, for the sizes where
    rep_fine_torch's [L, L + NB * RM + NB] graph does not fit: per query block one softmax over its tier-A tokens,
    its tier-B table rows with at least one member (+ ln of the member count) and its tier-C block means (+ ln of the
    block count) (reference experiments/vsa2_representative/vsa2_rep/reference.py:53-96). q, k, v, dout [L, D];
    masks [NB, NB]; tables = (k_mid, v_mid [NB * RM, D], k_tail, v_tail [NB, D]) as given values; groups [L] = the
    table row of each token (-1 on padding). delta = rowsum(dO * o_delta) (the stored O the backward consumes;
    this function's own O when None). Table gradients reach the tokens as the adjoint of a mean: row gradient /
    member count to each member, block-mean gradient / count to each valid token. Returns dict(o, lse, dq, dk, dv)
    and, for element bounds, the same products over absolute values (dq_abs, dk_abs, dv_abs: |dS| |K|, |dS|^T |Q|,
    P^T |dO| pushed through the same adjoints). Pinned against rep_fine_torch's autograd
    (tests/test_cpu_vsa_oracle.py)."""
    q, k, v, dout = (np.asarray(x, np.float64) for x in (q, k, v, dout))
    L, D = q.shape
    NB = L // BLOCK
    cnt = np.asarray(blk_cnt, np.int64)
    k_mid, v_mid, k_tail, v_tail = (np.asarray(t, np.float64) for t in tables)
    grp = np.asarray(groups, np.int64)
    ng = np.bincount(grp[grp >= 0], minlength=NB * RM)
    ma, mab = np.asarray(mask_a, bool), np.asarray(mask_ab, bool)
    sc = 1.0 / math.sqrt(D)
    o = np.zeros((L, D))
    lse = np.full(L, -np.inf)
    dq, dq_abs = np.zeros((L, D)), np.zeros((L, D))
    # gradients of every column source: tokens, table rows, block means (and their absolute-value twins)
    gk = [np.zeros((L, D)), np.zeros((NB * RM, D)), np.zeros((NB, D))]
    gv = [np.zeros_like(x) for x in gk]
    gk_abs = [np.zeros_like(x) for x in gk]
    gv_abs = [np.zeros_like(x) for x in gk]
    with np.errstate(divide="ignore"):
        ln_ng, ln_cnt = np.log(ng.astype(np.float64)), np.log(cnt.astype(np.float64))
    for i in range(NB):
        n = int(cnt[i])
        ja = np.nonzero(ma[i])[0]
        jb = np.nonzero(mab[i] & ~ma[i])[0]
        jc = np.nonzero(~mab[i])[0]
        tok = (np.concatenate([j * BLOCK + np.arange(cnt[j]) for j in ja]) if ja.size else np.zeros(0, np.int64))
        rows = (jb[:, None] * RM + np.arange(RM)[None, :]).reshape(-1)
        rows = rows[ng[rows] > 0]
        parts = ((0, tok), (1, rows), (2, jc))
        kc = np.concatenate([k[tok], k_mid[rows], k_tail[jc]])
        vc = np.concatenate([v[tok], v_mid[rows], v_tail[jc]])
        if n == 0 or kc.shape[0] == 0:
            continue
        bias = np.concatenate([np.zeros(tok.size), ln_ng[rows], ln_cnt[jc]])
        r = slice(i * BLOCK, i * BLOCK + n)
        s = q[r] @ kc.T * sc + bias[None, :]
        m = s.max(1, keepdims=True)
        lz = np.log(np.exp(s - m).sum(1, keepdims=True)) + m
        p = np.exp(s - lz)
        o[r] = p @ vc
        lse[r] = lz[:, 0]
        do = dout[r]
        delta = (do * (o[r] if o_delta is None else np.asarray(o_delta[r], np.float64))).sum(1, keepdims=True)
        ds = p * (do @ vc.T - delta)
        dq[r] = ds @ kc * sc
        dq_abs[r] = np.abs(ds) @ np.abs(kc) * sc
        dkc, dvc = ds.T @ q[r] * sc, p.T @ do
        dkc_abs, dvc_abs = np.abs(ds).T @ np.abs(q[r]) * sc, p.T @ np.abs(do)
        off = 0
        for src, idx in parts:
            sl = slice(off, off + idx.size)
            gk[src][idx] += dkc[sl]
            gv[src][idx] += dvc[sl]
            gk_abs[src][idx] += dkc_abs[sl]
            gv_abs[src][idx] += dvc_abs[sl]
            off += idx.size

    valid = grp >= 0
    blk = np.arange(L) // BLOCK
    g_ = np.where(valid, grp, 0)

    def tokens(acc):
        t, mid, tail = acc
        out = t.copy()
        out += np.where(valid[:, None], mid[g_] / np.maximum(ng[g_], 1)[:, None], 0)
        out += np.where(valid[:, None], tail[blk] / np.maximum(cnt[blk], 1)[:, None], 0)
        return out

    return dict(o=o, lse=lse, dq=dq, dk=tokens(gk), dv=tokens(gv), dq_abs=dq_abs, dk_abs=tokens(gk_abs),
                dv_abs=tokens(gv_abs))


def rep_kv_block_grads(q, k, v, dout, lse, delta, blk_cnt, mask_a, mask_ab, j, RM, tables, groups):
    """dK, dV [64, D] of the tokens of kv block j of ONE head in the three-tier attention, as a function of the
    backward's inputs: the forward's natural-log LSE [L] and delta = rowsum(dO * O) [L] of every query row (the
    values the backward kernels consume). Each query block i contributes through the one tier that holds j in row
    i: its tokens (tier A), its table rows with members (tier B, + ln of the member count, the row gradient shared
    by the members / count) or its block mean (tier C, + ln of the count, shared / count). Only the columns of
    block j are formed, so a full-size head costs O(L) products. Also returns the absolute-value products (|dS|^T
    |Q|, P^T |dO|) through the same adjoints, for element bounds. Pinned against rep_fine_head
    (tests/test_cpu_vsa_oracle.py)."""
    q, k, v, dout = (np.asarray(x, np.float64) for x in (q, k, v, dout))
    lse, delta = np.asarray(lse, np.float64), np.asarray(delta, np.float64)
    L, D = q.shape
    NB = L // BLOCK
    cnt = np.asarray(blk_cnt, np.int64)
    k_mid, v_mid, k_tail, v_tail = (np.asarray(t, np.float64) for t in tables)
    grp = np.asarray(groups, np.int64)
    ng = np.bincount(grp[grp >= 0], minlength=NB * RM)
    ma, mab = np.asarray(mask_a, bool), np.asarray(mask_ab, bool)
    sc = 1.0 / math.sqrt(D)
    n = int(cnt[j])
    tok = j * BLOCK + np.arange(n)
    rows_j = j * RM + np.arange(RM)
    rows_j = rows_j[ng[rows_j] > 0]
    dk, dv = np.zeros((BLOCK, D)), np.zeros((BLOCK, D))
    dk_abs, dv_abs = np.zeros((BLOCK, D)), np.zeros((BLOCK, D))

    def query_rows(which):
        qb = np.nonzero(which)[0]
        if qb.size == 0:
            return np.zeros(0, np.int64)
        return np.concatenate([i * BLOCK + np.arange(cnt[i]) for i in qb])

    def block(r, kc, vc, bias):
        s = q[r] @ kc.T * sc + bias[None, :]
        p = np.exp(s - lse[r][:, None])
        ds = p * (dout[r] @ vc.T - delta[r][:, None])
        return ds.T @ q[r] * sc, p.T @ dout[r], np.abs(ds).T @ np.abs(q[r]) * sc, p.T @ np.abs(dout[r])

    with np.errstate(divide="ignore"):
        # tier A: the block's tokens are columns of their own
        r = query_rows(ma[:, j])
        if r.size and n:
            a, b, c, d = block(r, k[tok], v[tok], np.zeros(n))
            dk[:n] += a
            dv[:n] += b
            dk_abs[:n] += c
            dv_abs[:n] += d
        # tier B: the table rows of block j, shared by their members
        r = query_rows(mab[:, j] & ~ma[:, j])
        if r.size and rows_j.size:
            a, b, c, d = block(r, k_mid[rows_j], v_mid[rows_j], np.log(ng[rows_j].astype(np.float64)))
            for x, y in ((dk, a), (dv, b), (dk_abs, c), (dv_abs, d)):
                for ri, row in enumerate(rows_j):
                    members = np.nonzero(grp[tok] == row)[0]
                    x[members] += y[ri] / ng[row]
        # tier C: the block mean, shared by every valid token
        r = query_rows(~mab[:, j])
        if r.size and n:
            a, b, c, d = block(r, k_tail[j:j + 1], v_tail[j:j + 1], np.log(np.array([float(n)])))
            for x, y in ((dk, a), (dv, b), (dk_abs, c), (dv_abs, d)):
                x[:n] += y[0] / n
    return dict(dk=dk, dv=dv, dk_abs=dk_abs, dv_abs=dv_abs)


def contiguous_groups(blk_cnt, RM):
    """Table row of every token for the contiguous groups of 64 / RM tokens (-1 on padding)."""
    cnt = np.asarray(blk_cnt, np.int64)
    L = cnt.size * BLOCK
    t = np.arange(L)
    return np.where(token_valid(cnt, L), (t // BLOCK) * RM + (t % BLOCK) // (BLOCK // RM), -1)


# --------------------------------------------------------------------- seeded k-means representative tables
# Not in the reference (its tables are contiguous group means, vsa2_rep/reference.py:23-50); this is the
# construction the HunyuanVideo-shape three-tier benchmark names ("tables built from seeded k-means, 5 iterations"), defined here and
# built by vsa_rep_build_kmeans. The arithmetic is float32 in a fixed order with no fused multiply-add, so the GPU
# tables, counts and labels equal these bit for bit.
_M32 = 0xFFFFFFFF


def _fmix32(h):
    """MurmurHash3's 32-bit finaliser (on Python ints, kept to 32 bits)."""
    h &= _M32
    h ^= h >> 16
    h = (h * 0x85EBCA6B) & _M32
    h ^= h >> 13
    h = (h * 0xC2B2AE35) & _M32
    h ^= h >> 16
    return h


def kmeans_seed_tokens(seed, bh, blk, n, RM):
    """The tokens of a block of n valid tokens that seed its min(RM, n) clusters: a partial Fisher-Yates shuffle of
    0..n-1 whose i-th swap partner is i + h_i mod (n - i), h_i = fmix32(seed * 0x9E3779B9 ^ fmix32(bh * 0x85EBCA6B ^
    fmix32(blk * 0xC2B2AE35 ^ i)))."""
    perm = list(range(n))
    for i in range(min(RM, n)):
        h = _fmix32((seed * 0x9E3779B9) ^ _fmix32((bh * 0x85EBCA6B) ^ _fmix32((blk * 0xC2B2AE35) ^ i)))
        j = i + h % (n - i)
        perm[i], perm[j] = perm[j], perm[i]
    return perm[:min(RM, n)]


def kmeans_tables(k, v, blk_cnt, RM, iters=5, seed=0, rnd=round_bf16, bh0=0, blk0=0):
    """Seeded Lloyd k-means of every block's valid keys into RM clusters: (k_mid, v_mid [B, H, NB * RM, D] rnd-ed
    cluster means (zero rows for empty clusters), lc_mid [B, H, NB * RM] log2 counts (-inf when empty), counts
    [B, H, NB * RM] int, labels [B, H, L] int (-1 on padding)).

    Per block: centroids start at the seed tokens' keys (clusters past n stay empty); each of `iters` rounds
    assigns every valid token to its nearest centroid (squared distance summed over the D columns in order,
    float32, each difference squared then added; ties to the smaller cluster) and moves every non-empty cluster's
    centroid to the float32 mean of its members' keys (summed in token order, then one division). The tables hold
    the last round's centroids and the mean values of the same clusters. bh0 / blk0: the (b, h) and block index of
    the first given head / block (the seeds depend on them), to check samples of a larger tensor."""
    k, v = np.asarray(k, np.float32), np.asarray(v, np.float32)
    B, H, L, D = k.shape
    NB = L // BLOCK
    cnt = np.asarray(blk_cnt, np.int64)
    k_mid = np.zeros((B, H, NB * RM, D), np.float32)
    v_mid = np.zeros_like(k_mid)
    counts = np.zeros((B, H, NB * RM), np.int64)
    labels = np.full((B, H, L), -1, np.int64)
    for b in range(B):
        for h in range(H):
            bh = bh0 + b * H + h
            for blk in range(NB):
                n = int(cnt[blk])
                x = k[b, h, blk * BLOCK:blk * BLOCK + n]
                seeds = kmeans_seed_tokens(seed, bh, blk0 + blk, n, RM)
                cent = np.zeros((RM, D), np.float32)
                cent[:len(seeds)] = x[seeds]
                live = np.arange(RM) < len(seeds)
                lab = np.zeros(n, np.int64)
                for _ in range(iters):
                    dist = np.zeros((n, RM), np.float32)
                    for d in range(D):
                        diff = (x[:, d:d + 1] - cent[None, :, d]).astype(np.float32)
                        dist = (dist + (diff * diff).astype(np.float32)).astype(np.float32)
                    dist[:, ~live] = np.inf
                    lab = np.argmin(dist, axis=1)          # first minimum: ties to the smaller cluster
                    for c in range(RM):
                        members = np.nonzero(lab == c)[0]
                        if members.size:
                            s = np.zeros(D, np.float32)
                            for t in members:
                                s = (s + x[t]).astype(np.float32)
                            cent[c] = (s / np.float32(members.size)).astype(np.float32)
                y = v[b, h, blk * BLOCK:blk * BLOCK + n]
                for c in range(RM):
                    members = np.nonzero(lab == c)[0]
                    row = blk * RM + c
                    counts[b, h, row] = members.size
                    if members.size:
                        s = np.zeros(D, np.float32)
                        for t in members:
                            s = (s + y[t]).astype(np.float32)
                        k_mid[b, h, row] = rnd(cent[c])
                        v_mid[b, h, row] = rnd((s / np.float32(members.size)).astype(np.float32))
                labels[b, h, blk * BLOCK:blk * BLOCK + n] = lab
    with np.errstate(divide="ignore"):
        lc = np.where(counts > 0, np.log2(np.maximum(counts, 1).astype(np.float64)), -np.inf)
    return k_mid, v_mid, lc, counts, labels


def row_tiers(scores, ka, kab):
    """Per-query-block tier split (the three-tier benchmark's wording; the reference splits by two global budgets,
    vsa2_rep/ops.py:50-85): tier A = the min(ka, NB) best kv blocks of each row, A|B = the min(kab, NB) best, under
    row_topk_mask's order (score desc, ties to the smaller index). Returns the two bool masks."""
    return row_topk_mask(scores, ka), row_topk_mask(scores, max(ka, kab))
