"""Three-tier (64 / 4 / 1) forward and backward at NB = 600 against the blockwise float64 oracle
(oracle/vsa_ref.py::rep_fine_head) over a whole head: O, LSE, dQ, dK and dV of every token. At NB > 256 the table
gradient kernel refills its list of query blocks to visit (256 at a time) several times per row group, a path the
NB = 10 tests do not reach. Both constructions: the reference's (global budgets, contiguous group means) and the
three-tier benchmark's (per-query-block tiers, seeded k-means tables). The oracle uses the kernels' own bf16 tables
(pinned bit for bit elsewhere) and delta from the stored bf16 O, the values the backward consumes.

Tolerances: O and LSE max-abs 2e-2 / rel-L2 1e-2. Gradients: rel-L2 1e-2, and per element the larger of 2e-2 and
twice the rounding the kernels' arithmetic allows: dS enters the MFMA products as bf16 (relative error <= 2^-9 per
element) and the gradients are stored as bf16, so |err| <= 2^-9 (|dS| |K| scale + |dQ|) for dQ, and the same with
|dS|^T |Q| for dK and P^T |dO| for dV; the bound is 2^-8 times those sums."""
import math
import sys

import numpy as np
import pytest
import torch

from helpers import check_close, f32
from oracle import vsa_ref as ref

pytestmark = pytest.mark.gpu

B, H, D, RM = 1, 2, 128, 4
NB = 600
TAIL = 44
L = NB * 64


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def check_grad(name, got, want, absum):
    err = np.abs(got - want)
    bound = np.maximum(2e-2, 2.0 ** -8 * (absum + np.abs(want)))
    log(f"{name}: max-abs {err.max():.3g}, worst err / bound {float((err / bound).max()):.3g}")
    assert (err <= bound).all(), f"{name}: worst err / bound {float((err / bound).max()):.3g}"
    check_close(name, got, want, max_abs=np.inf)


@pytest.mark.parametrize("construction", ["reference", "baseline"])
def test_three_tier_backward_with_list_refills(dev, construction):
    from self_trainable_or_free_attn_amd.vsa import _C, rep
    log("NB 600 three tiers:", construction)
    cnt = np.full(NB, 64)
    cnt[-1] = TAIL
    valid = torch.as_tensor(ref.token_valid(cnt, L))[None, None, :, None]
    g = torch.Generator().manual_seed(31)
    q, k, v, dout = ((torch.randn(B, H, L, D, generator=g) * valid).to(torch.bfloat16) for _ in range(4))
    qd, kd, vd, dod = (x.to(dev) for x in (q, k, v, dout))
    blk = torch.as_tensor(cnt, dtype=torch.int32, device=dev)
    kmeans = construction == "baseline"
    tiers = rep.RepTiers(frac_full=0.05, frac_mid=0.20, mid_reps=RM, split="per_row" if kmeans else "global",
                         tables="kmeans" if kmeans else "contiguous", kmeans_iters=5, seed=4)
    sel = rep.route_tiers(qd, kd, blk, tiers, R=16)
    x = [t.detach().clone().requires_grad_(True) for t in (qd, kd, vd)]
    o, lse = rep.rep_fine_attention(*x, blk, sel, mid_reps=RM, tables=tiers.tables, kmeans_iters=5, seed=4)
    grads = torch.autograd.grad(o, x, dod)
    if kmeans:
        (k_mid, v_mid, _, k_tail, v_tail, _), counts, labels = _C.rep_build_kmeans(kd, vd, blk, RM, 5, 4)
    else:
        k_mid, v_mid, _, k_tail, v_tail, _ = _C.rep_build(kd, vd, blk, RM)
    torch.cuda.synchronize()
    ma, mb, _ = (m.cpu().numpy() for m in sel.tier_masks(NB))
    go, gl = f32(o), f32(lse)
    gq, gk, gv = (f32(t) for t in grads)
    for h in range(H):
        log("NB 600 three tiers:", construction, "oracle of head", h)
        if kmeans:
            lab = labels[0, h].cpu().numpy().astype(np.int64)
            groups = np.where(ref.token_valid(cnt, L), (np.arange(L) // 64) * RM + lab, -1)
            assert np.array_equal(np.bincount(groups[groups >= 0], minlength=NB * RM),
                                  counts[0, h].cpu().numpy())
        else:
            groups = ref.contiguous_groups(cnt, RM)
        tables = [f32(t[0, h, :n]).astype(np.float64) for t, n in
                  ((k_mid, NB * RM), (v_mid, NB * RM), (k_tail, NB), (v_tail, NB))]
        want = ref.rep_fine_head(f32(q[0, h]), f32(k[0, h]), f32(v[0, h]), cnt, ma[0, h], ma[0, h] | mb[0, h], RM,
                                 tables, groups, f32(dout[0, h]), o_delta=go[0, h])
        check_close(f"O h{h}", go[0, h], want["o"])
        fin = np.isfinite(want["lse"])
        assert np.array_equal(np.isfinite(gl[0, h]), fin)
        check_close(f"LSE h{h}", gl[0, h][fin], want["lse"][fin])
        check_grad(f"dQ h{h}", gq[0, h], want["dq"], want["dq_abs"])
        check_grad(f"dK h{h}", gk[0, h], want["dk"], want["dk_abs"])
        check_grad(f"dV h{h}", gv[0, h], want["dv"], want["dv_abs"])
