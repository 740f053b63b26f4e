"""VSA routing and three-tier attention beyond 2048 blocks (longer videos than the HunyuanVideo benchmark clip):
* byte for byte against the oracle: the original-VSA router (block scores and per-row top-K, 8 rows per workgroup
  past 2048 blocks) at NB = 2049, 3000 and 5000, bf16 and fp16; the exact global top-k and the kv->q inversion at
  NB = 4200; the per-query-block tiers at NB = 3000 and 5000 (the 64- and 128-chunk register layouts);
* the three-tier forward / backward at NB = 3000 (192 000 tokens, a 40-token tail block) in both constructions and
  at NB = 4500 (the 8192-entry block lists): O / LSE / dQ of sampled query blocks and dK / dV of sampled kv blocks
  against the float64 oracle (oracle/vsa_ref.py rep_fine_head restated per block, and rep_kv_block_grads), max-abs
  2e-2 / rel-L2 1e-2 with the gradients' conditioning bound (see tests/test_gpu_vsa_rep_backward_sizes.py)."""
import math
import sys

import numpy as np
import pytest
import torch

from helpers import check_close, f32
from oracle import vsa_ref as ref

pytestmark = pytest.mark.gpu


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def C():
    from self_trainable_or_free_attn_amd.vsa import _C
    return _C


def head_csr(mask, base):
    counts = mask.sum(1)
    return (base + np.concatenate([[0], np.cumsum(counts)])).astype(np.int64), np.nonzero(mask)[1].astype(np.int64)


def bitmap(mask):
    nb = mask.shape[-1]
    w = (nb + 31) // 32
    m = np.zeros((nb, w * 32), bool)
    m[:, :nb] = mask
    return (m.reshape(nb, w, 32).astype(np.uint64) << np.arange(32, dtype=np.uint64)).sum(-1).astype(np.uint32) \
        .view(np.int32)


def check_csr(q2k_ptr, q2k_idx, k2q_ptr, k2q_idx, mask):
    qp, qi, kp, ki = (x.cpu().numpy() for x in (q2k_ptr, q2k_idx, k2q_ptr, k2q_idx))
    rp, ri = ref.csr_from_mask(mask)
    assert np.array_equal(qp, rp) and np.array_equal(qi[:ri.size], ri), "q2k lists differ"
    cp, ci = ref.csr_from_mask(np.swapaxes(mask, -1, -2))
    assert np.array_equal(kp, cp) and np.array_equal(ki[:ci.size], ci), "k2q lists differ"


@pytest.mark.parametrize("NB,K,dtype", [(2049, 2049, "bf16"), (2049, 0, "bf16"), (3000, 150, "bf16"),
                                         (5000, 61, "bf16"), (3000, 150, "f16")])
def test_route_rows_beyond_2048(dev, NB, K, dtype):
    from oracle.bf16 import round_bf16, round_f16
    B, H, D = 1, 2, 128
    log("route_rows NB", NB, "K", K, dtype)
    g = torch.Generator().manual_seed(NB + K)
    pad = -(-NB // 64) * 64
    tdt, rnd = (torch.bfloat16, round_bf16) if dtype == "bf16" else (torch.float16, round_f16)
    qc, kc = ((torch.randn(B, H, pad, D, generator=g) * 0.5).to(tdt).to(dev) for _ in range(2))
    scores = C().block_scores(qc, kc, NB)
    got = C().route_rows(qc, kc, NB, K)
    torch.cuda.synchronize()
    gs = f32(scores)
    # the scores of the wide path against the float64 op: the GPU's fp32 dot differs from the exact one by at most
    # n u sum|q k| (n = 128 terms, u = 2^-24), and the two bf16 roundings then land at most one step further each
    h = 1
    rows = np.r_[0:40, NB - 40:NB]
    qh, kh = f32(qc)[0, h, rows].astype(np.float64), f32(kc)[0, h, :NB].astype(np.float64)
    want_s = ref.block_scores(qh, kh, rnd=rnd)
    mant = 7 if dtype == "bf16" else 10
    step = np.exp2(np.floor(np.log2(np.maximum(np.abs(want_s), 2.0 ** -100))) - mant)
    dot_err = D * 2.0 ** -24 * (np.abs(qh) @ np.abs(kh).T) / np.sqrt(D)
    assert (np.abs(gs[h, rows] - want_s) <= 2 * step + dot_err).all()
    assert (gs[h, rows] == want_s).mean() > 0.95
    check_csr(*got, ref.row_topk_mask(gs.reshape(B, H, NB, NB), K))


def test_row_topk_beyond_2048_with_ties(dev):
    NB, K = 5000, 700
    log("row_topk NB", NB, "K", K)
    g = torch.Generator().manual_seed(9)
    s = (torch.randint(-24, 24, (2, NB, NB), generator=g).float() / 8).to(torch.bfloat16)
    s[0, 3] = -0.0
    s[1, :, 17] = 0.0
    i32 = dict(device=dev, dtype=torch.int32)
    out = [torch.empty(1, 2, NB + 1, **i32), torch.empty(2 * NB * K, **i32), torch.empty(1, 2, NB + 1, **i32),
           torch.empty(2 * NB * K, **i32)]
    C().row_topk_into(s.to(dev), K, 0, *out)
    torch.cuda.synchronize()
    check_csr(*out, ref.row_topk_mask(f32(s).reshape(1, 2, NB, NB), K))


def test_global_topk_and_inversion_beyond_4096(dev):
    NB = 4200
    g = np.random.default_rng(42)
    scores = (g.integers(0, 4096, (1, NB, NB)) / 4096.0).astype(np.float32)   # many ties
    budget = int(0.05 * NB * NB)
    log("global top-k NB", NB, "budget", budget)
    out = [torch.empty(1, 1, NB + 1, dtype=torch.int32, device=dev), torch.empty(budget, dtype=torch.int32, device=dev),
           torch.empty(1, 1, NB + 1, dtype=torch.int32, device=dev), torch.empty(budget, dtype=torch.int32, device=dev)]
    C().global_topk_into(torch.from_numpy(scores).to(dev), budget, 0, *out)
    qp, qi, kp, ki = (x.cpu().numpy() for x in out)
    order = ref._desc_order(scores.reshape(-1))
    m = np.zeros(NB * NB, bool)
    m[order[:budget]] = True
    m = m.reshape(NB, NB)
    wp, wi = head_csr(m, 0)
    assert np.array_equal(qp[0, 0], wp) and np.array_equal(qi, wi)
    wp, wi = head_csr(m.T, 0)
    assert np.array_equal(kp[0, 0], wp) and np.array_equal(ki, wi)


@pytest.mark.parametrize("NB", [3000, 5000])
def test_row_tiers_beyond_2048(dev, NB):
    from self_trainable_or_free_attn_amd import _lib
    g = np.random.default_rng(NB)
    scores = (g.integers(0, 1024, (1, NB, NB)) / 1024.0 - 0.5).astype(np.float32)
    scores[0, 7] = -0.0
    ka, kab = int(round(0.05 * NB)), int(round(0.25 * NB))
    log("row tiers NB", NB)
    W = (NB + 31) // 32
    i32 = dict(device=dev, dtype=torch.int32)
    a_ptr, ab_ptr = torch.empty(1, 1, NB + 1, **i32), torch.empty(1, 1, NB + 1, **i32)
    a_idx, ab_idx = torch.empty(NB * ka, **i32), torch.empty(NB * kab, **i32)
    bits_a, bits_ab = torch.zeros(1, 1, NB, W, **i32), torch.zeros(1, 1, NB, W, **i32)
    _lib.call("vsa_row_tiers", torch.from_numpy(scores).to(dev), NB, 0, 1, ka, kab, a_ptr, a_idx, ab_ptr, ab_idx,
              bits_a, bits_ab)
    torch.cuda.synchronize()
    ma, mab = ref.row_tiers(scores[0], ka, kab)
    assert np.array_equal(bits_a.cpu().numpy()[0, 0], bitmap(ma))
    assert np.array_equal(bits_ab.cpu().numpy()[0, 0], bitmap(mab))
    wp, wi = head_csr(ma, 0)
    assert np.array_equal(a_ptr.cpu().numpy()[0, 0], wp) and np.array_equal(a_idx.cpu().numpy(), wi)
    wp, wi = head_csr(mab, 0)
    assert np.array_equal(ab_ptr.cpu().numpy()[0, 0], wp) and np.array_equal(ab_idx.cpu().numpy(), wi)


def _block_oracle(q, k, v, dout, go, cnt, ma, mab, RM, tables, groups, i):
    """O, LSE, dQ of query block i and the element bound of dQ (float64, the block's own columns)."""
    k_mid, v_mid, k_tail, v_tail = tables
    ng = np.bincount(groups[groups >= 0], minlength=len(cnt) * RM)
    ja, jb, jc = np.nonzero(ma[i])[0], np.nonzero(mab[i] & ~ma[i])[0], np.nonzero(~mab[i])[0]
    tok = np.concatenate([j * 64 + np.arange(cnt[j]) for j in ja]) if ja.size else np.zeros(0, np.int64)
    rows = (jb[:, None] * RM + np.arange(RM)[None, :]).reshape(-1)
    rows = rows[ng[rows] > 0]
    kc = np.concatenate([k[tok], k_mid[rows], k_tail[jc]])
    vc = np.concatenate([v[tok], v_mid[rows], v_tail[jc]])
    bias = np.concatenate([np.zeros(tok.size), np.log(ng[rows]), np.log(cnt[jc].astype(np.float64))])
    r = slice(i * 64, i * 64 + int(cnt[i]))
    sc = 1.0 / math.sqrt(q.shape[1])
    s = q[r] @ kc.T * sc + bias[None, :]
    m = s.max(1, keepdims=True)
    lz = np.log(np.exp(s - m).sum(1, keepdims=True)) + m
    p = np.exp(s - lz)
    dlt = (dout[r] * go[r]).sum(1, keepdims=True)
    ds = p * (dout[r] @ vc.T - dlt)
    dq = ds @ kc * sc
    return p @ vc, lz[:, 0], dq, np.abs(ds) @ np.abs(kc) * sc


def check_bound(name, got, want, absum):
    err = np.abs(got - want)
    bound = np.maximum(2e-2, 2.0 ** -8 * (absum + np.abs(want)))
    log(f"{name}: max-abs {err.max():.3g}")
    assert (err <= bound).all(), f"{name}: worst err / bound {float((err / bound).max()):.3g}"
    check_close(name, got, want, max_abs=np.inf)


@pytest.mark.parametrize("NB,construction", [(3000, "reference"), (3000, "baseline"), (4500, "reference")])
def test_three_tiers_beyond_2048(dev, NB, construction):
    """NB = 4500 takes the forward / dQ kernels' 8192-entry block lists (one workgroup per CU)."""
    from self_trainable_or_free_attn_amd.vsa import _C, rep
    B, H, D, RM = 1, 2, 128, 4
    cnt = np.full(NB, 64)
    cnt[-1] = 40
    L = NB * 64
    valid = torch.as_tensor(ref.token_valid(cnt, L))[None, None, :, None]
    g = torch.Generator().manual_seed(77)
    q, k, v, dout = ((torch.randn(B, H, L, D, generator=g) * valid).to(torch.bfloat16) for _ in range(4))
    qd, kd, vd, dod = (x.to(dev) for x in (q, k, v, dout))
    blk = torch.as_tensor(cnt, dtype=torch.int32, device=dev)
    kmeans = construction == "baseline"
    tiers = rep.RepTiers(frac_full=0.05, frac_mid=0.20, mid_reps=RM, split="per_row" if kmeans else "global",
                         tables="kmeans" if kmeans else "contiguous", kmeans_iters=5, seed=3)
    log("NB", NB, "three tiers:", construction)
    sel = rep.route_tiers(qd, kd, blk, tiers, R=16)
    x = [t.detach().clone().requires_grad_(True) for t in (qd, kd, vd)]
    o, lse = rep.rep_fine_attention(*x, blk, sel, mid_reps=RM, tables=tiers.tables, kmeans_iters=5, seed=3)
    gq, gk, gv = (f32(t) for t in torch.autograd.grad(o, x, dod))
    if kmeans:
        (k_mid, v_mid, _, k_tail, v_tail, _), counts, labels = _C.rep_build_kmeans(kd, vd, blk, RM, 5, 3)
    else:
        k_mid, v_mid, _, k_tail, v_tail, _ = _C.rep_build(kd, vd, blk, RM)
    torch.cuda.synchronize()
    ma, mb, _ = (m.cpu().numpy() for m in sel.tier_masks(NB))
    go, gl = f32(o), f32(lse)
    for h in range(H):
        if kmeans:
            lab = labels[0, h].cpu().numpy().astype(np.int64)
            groups = np.where(ref.token_valid(cnt, L), (np.arange(L) // 64) * RM + lab, -1)
        else:
            groups = ref.contiguous_groups(cnt, RM)
        tables = [f32(t[0, h, :n]).astype(np.float64) for t, n in
                  ((k_mid, NB * RM), (v_mid, NB * RM), (k_tail, NB), (v_tail, NB))]
        qh, kh, vh, dh = (f32(t[0, h]).astype(np.float64) for t in (q, k, v, dout))
        mah, mabh = ma[0, h], ma[0, h] | mb[0, h]
        for i in (0, 1777, NB - 1):
            log("NB", NB, construction, "head", h, "query block", i)
            wo, wl, wdq, bq = _block_oracle(qh, kh, vh, dh, go[0, h], cnt, mah, mabh, RM, tables, groups, i)
            r = slice(i * 64, i * 64 + int(cnt[i]))
            check_close(f"O h{h} b{i}", go[0, h, r], wo)
            check_close(f"LSE h{h} b{i}", gl[0, h, r], wl)
            check_bound(f"dQ h{h} b{i}", gq[0, h, r], wdq, bq)
        dlt = (dh * go[0, h]).sum(1)
        for j in (5, 2222, NB - 1):
            w = ref.rep_kv_block_grads(qh, kh, vh, dh, np.where(np.isfinite(gl[0, h]), gl[0, h], 0.0), dlt, cnt,
                                       mah, mabh, j, RM, tables, groups)
            n = int(cnt[j])
            check_bound(f"dK h{h} kv{j}", gk[0, h, j * 64:j * 64 + n], w["dk"][:n], w["dk_abs"][:n])
            check_bound(f"dV h{h} kv{j}", gv[0, h, j * 64:j * 64 + n], w["dv"][:n], w["dv_abs"][:n])
