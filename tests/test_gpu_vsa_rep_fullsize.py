"""VSA2 three tiers (64 / 4 / 1) at the full C4 HunyuanVideo shape (B = 2, H = 24, 33 x 45 x 80 grid = 118 800
tokens in 1857 blocks, a 16-token tail block, D = 128; tiers 5 % full, 20 % as 4 representatives, the rest block
means; the benchmark's inputs), in both constructions: the reference's (two global budgets, contiguous group
means) and the benchmark's (per-query-block tiers, seeded 5-round k-means tables; sampled table blocks equal
the oracle's bit for bit). Checked: the forward output, LSE and dQ of sampled query blocks against a float64
restatement of one softmax over the block's tier-A tokens, tier-B representatives (+ ln of the group size) and
tier-C block means (+ ln of the block count; dQ with delta = rowsum(dO * O) of the stored bf16 O, the quantity the
backward consumes), with the kernels' own bf16 tables (`vsa_rep_build`, bit-exact at
small sizes) and tier bitmaps; max-abs 2e-2 / rel-L2 1e-2 (dQ: rel-L2 1e-2 and an element
bound from the conditioning of the bf16 dS sum, see below). dK / dV of the sampled blocks' tokens, over every query
block of the head (oracle/vsa_ref.py::rep_kv_block_grads from the stored LSE and delta), under the same kind of
bound."""
import math
import sys

import numpy as np
import pytest
import torch

from helpers import check_close, f32
from oracle import vsa_ref

pytestmark = pytest.mark.gpu

GRID = (33, 45, 80)
B, H, D, RM = 2, 24, 128, 4
SAMPLES = [(0, 0, 0), (1, 13, 900), (1, 23, 1856)]  # (batch, head, query block); block 1856 is the tail


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("construction", ["reference", "baseline"])
def test_three_tiers_full_c4_shape(dev, construction):
    from self_trainable_or_free_attn_amd import synthetic
    from self_trainable_or_free_attn_amd.vsa import _C, rep
    log("C4 full shape: inputs")
    Lr = GRID[0] * GRID[1] * GRID[2]
    NB = -(-Lr // 64)
    xs = []
    for b in range(B):
        qb, kb, vb, _ = synthetic.fourier_qkv(GRID, H, D, seed=21 + b, device=dev, pad_to=NB * 64)
        xs.append([t.permute(1, 0, 2) for t in (qb, kb, vb)])
    q, k, v = (torch.stack([x[i] for x in xs]).contiguous() for i in range(3))
    del xs
    blk = torch.full((NB,), 64, dtype=torch.int32, device=dev)
    blk[-1] = Lr - 64 * (NB - 1)
    g = torch.Generator(device=dev).manual_seed(5)
    dout = torch.randn(q.shape, device=dev, generator=g).to(torch.bfloat16)
    kmeans = construction == "baseline"
    tiers = rep.RepTiers(frac_full=0.05, frac_mid=0.20, mid_reps=RM, split="per_row" if kmeans else "global",
                         tables="kmeans" if kmeans else "contiguous", kmeans_iters=5, seed=4)
    sel = rep.route_tiers(q, k, blk, tiers, R=16)
    log("C4 full shape:", construction, "kernels")
    qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o, lse = rep.rep_fine_attention(qg, kg, vg, blk, sel, mid_reps=RM, tables=tiers.tables, kmeans_iters=5, seed=4)
    dq, dk, dv = torch.autograd.grad(o, (qg, kg, vg), dout)
    del qg, kg, vg
    cnt = blk.cpu().numpy().astype(np.int64)
    if kmeans:
        (k_mid, v_mid, _, k_tail, v_tail, _), counts, labels = _C.rep_build_kmeans(k, v, blk, RM, 5, 4)
        ng_all = counts.cpu().numpy().reshape(B, H, NB, RM)                 # cluster sizes per (b, h)
    else:
        k_mid, v_mid, _, k_tail, v_tail, _ = _C.rep_build(k, v, blk, RM)
        gs = 64 // RM
        ng_all = np.broadcast_to(np.clip(cnt[:, None] - np.arange(RM)[None, :] * gs, 0, gs), (B, H, NB, RM))
    torch.cuda.synchronize()
    ma, mb, mc = (m.cpu().numpy() for m in sel.tier_masks(NB))
    if kmeans:
        ka, kab = tiers.row_budgets(NB)
        assert (ma.sum(-1) == ka).all() and ((ma | mb).sum(-1) == kab).all()
    sc = 1.0 / math.sqrt(D)
    go, gl, gdq = f32(o), f32(lse), f32(dq)
    for b, h, i in SAMPLES:
        log("C4 full shape: oracle batch", b, "head", h, "block", i)
        ng = ng_all[b, h]
        if kmeans:   # the sampled block's k-means table rows against the oracle (same seed, same (b, h, block))
            sl = slice(i * 64, i * 64 + 64)
            wk, wv, _, wc, _ = vsa_ref.kmeans_tables(f32(k[b, h, sl])[None, None], f32(v[b, h, sl])[None, None],
                                                     [int(cnt[i])], RM, 5, 4, bh0=b * H + h, blk0=i)
            assert np.array_equal(ng[i], wc[0, 0])
            assert np.array_equal(f32(k_mid[b, h, i * RM:(i + 1) * RM]), wk[0, 0])
            assert np.array_equal(f32(v_mid[b, h, i * RM:(i + 1) * RM]), wv[0, 0])
        kh, vh = k[b, h].double().cpu().numpy(), v[b, h].double().cpu().numpy()
        kmid, vmid = k_mid[b, h].double().cpu().numpy(), v_mid[b, h].double().cpu().numpy()
        ktail, vtail = k_tail[b, h].double().cpu().numpy(), v_tail[b, h].double().cpu().numpy()
        ja, jb, jc = (np.nonzero(m[b, h, i])[0] for m in (ma, mb, mc))
        tok = np.concatenate([j * 64 + np.arange(cnt[j]) for j in ja]) if ja.size else np.zeros(0, np.int64)
        grp = np.array([j * RM + r for j in jb for r in range(RM) if ng[j, r] > 0], np.int64)
        kc = np.concatenate([kh[tok], kmid[grp], ktail[jc]])
        vc = np.concatenate([vh[tok], vmid[grp], vtail[jc]])
        bias = np.concatenate([np.zeros(tok.size), np.log(ng.reshape(-1)[grp]), np.log(cnt[jc])])
        rows = slice(i * 64, i * 64 + int(cnt[i]))
        qi = q[b, h, rows].double().cpu().numpy()
        s = qi @ kc.T * sc + bias[None, :]
        m = s.max(1, keepdims=True)
        lz = np.log(np.exp(s - m).sum(1, keepdims=True)) + m
        p = np.exp(s - lz)
        out = p @ vc
        check_close(f"O b{b} h{h} blk{i}", go[b, h, rows], out)
        check_close(f"LSE b{b} h{h} blk{i}", gl[b, h, rows], lz[:, 0])
        doi = dout[b, h, rows].double().cpu().numpy()
        # delta = rowsum(dO * O) from the stored bf16 O, as the backward kernels (and the reference's) form it
        dlt = (doi * go[b, h, rows]).sum(1, keepdims=True)
        ds = p * (doi @ vc.T - dlt)
        want_dq = ds @ kc * sc
        check_close(f"dQ b{b} h{h} blk{i}", gdq[b, h, rows], want_dq, max_abs=np.inf)
        # element bound from the conditioning of the sum: dS enters the MFMA as bf16 (round-to-nearest, relative
        # error <= 2^-9 per element) and dQ is stored as bf16, so |err| <= 2^-9 * (|dS| @ |K|) * scale + 2^-9 |dQ|;
        # the bound below is twice that (and never under 2e-2). Rows where ~3 000 columns nearly cancel reach
        # 0.04 here while the plain 2e-2 bound holds elsewhere.
        bound = np.maximum(2e-2, 2.0 ** -8 * ((np.abs(ds) @ np.abs(kc)) * sc + np.abs(want_dq)))
        err = np.abs(gdq[b, h, rows] - want_dq)
        assert (err <= bound).all(), f"dQ b{b} h{h} blk{i}: worst err / bound {float((err / bound).max()):.3g}"
        if int(cnt[i]) < 64:
            assert (go[b, h, i * 64 + int(cnt[i]):(i + 1) * 64] == 0).all()
        # dK / dV of kv block i of this head (its tokens, and through the adjoints its tier-B table rows and its
        # block mean), over every query block of the head, from the backward's inputs: the stored LSE and
        # delta = rowsum(dO * O) of the bf16 O; same element bound with |dS|^T |Q| and P^T |dO|
        if kmeans:
            lab = labels[b, h].cpu().numpy().astype(np.int64)
            groups = np.where(lab < RM, (np.arange(NB * 64) // 64) * RM + lab, -1)
        else:
            groups = vsa_ref.contiguous_groups(cnt, RM)
        dlt_all = (dout[b, h].double().cpu().numpy() * go[b, h]).sum(1)
        wkv = vsa_ref.rep_kv_block_grads(q[b, h].float().cpu().numpy(), k[b, h].float().cpu().numpy(),
                                         v[b, h].float().cpu().numpy(), dout[b, h].float().cpu().numpy(),
                                         np.where(np.isfinite(gl[b, h]), gl[b, h], 0.0), dlt_all, cnt, ma[b, h],
                                         ma[b, h] | mb[b, h], i, RM, (kmid[:NB * RM], vmid[:NB * RM], ktail[:NB],
                                                                     vtail[:NB]), groups)
        n = int(cnt[i])
        for name, got, key in (("dK", dk, "dk"), ("dV", dv, "dv")):
            g_ = f32(got[b, h, i * 64:i * 64 + n])
            w_ = wkv[key][:n]
            bound = np.maximum(2e-2, 2.0 ** -8 * (wkv[key + "_abs"][:n] + np.abs(w_)))
            err = np.abs(g_ - w_)
            log(f"C4 {name} b{b} h{h} blk{i}: max-abs {err.max():.3g}")
            assert (err <= bound).all(), f"{name} b{b} h{h} blk{i}: worst err / bound {float((err / bound).max()):.3g}"
            check_close(f"{name} b{b} h{h} blk{i}", g_, w_, max_abs=np.inf)
