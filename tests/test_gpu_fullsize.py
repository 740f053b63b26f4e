"""The sparse step at the full Wan2.1-14B shape (L = 75 600 = 1182 kv blocks, 591 query tiles with an 80-row tail
tile, H = 40, D = 128, density 0.10), through the production pipeline with two CFG branches (dense step, full
step, then the sparse step: branch 0 with the kernel-built plan, branch 1 on the same plan with its own block
means, representatives, offset and flags), checked against the CPU oracle on sampled (tile, head) pairs. The oracle
evaluates exactly the same column lists, so the checks cover 32-bit addressing over the full tensors, long lists
through the staged list ring, the tail tile and the mass map at full size, at max-abs 2e-2 / rel-L2 1e-2 (mass: 2e-2
of its largest value):

* branch 0: a direct launch on the pipeline's lists and state (O, LSE, flag, mass);
* branch 1: the pipeline's own output of its call (the fixed-offset result, or the fallback + compensation
  result where its flag is set), its LSE (the offset it leaves) and flags;
* forced fallback at full size: the offset shifted by +200 (reference tests/test_attention.py:141-149) flags every
  tile, and the online fallback over the list plus the block-mean compensation are checked."""
import sys

import numpy as np
import pytest
import torch

from helpers import check_close, f32
from oracle import echosparse_ref as ref

pytestmark = pytest.mark.gpu

GRID = (21, 45, 80)
H, D, BM = 40, 128, 128
# (query tile, head); tile 590 is the 80-row tail tile
PAIRS = [(0, 0), (295, 17), (590, 39), (123, 5), (37, 1), (200, 22), (333, 30), (401, 8), (480, 13), (555, 27),
         (590, 2), (17, 36)]
PAIRS_B1 = [(0, 3), (150, 19), (590, 11), (444, 38), (77, 24), (301, 6)]
PAIRS_FALLBACK = [(1, 9), (312, 31), (590, 20), (250, 0)]


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def wan(dev):
    from self_trainable_or_free_attn_amd import EchoSparseAttention, synthetic
    log("full-size sparse step: building Wan-shaped inputs")
    q, k, v, _ = synthetic.fourier_qkv(GRID, H, D, seed=11, device=dev)
    clean = [(q, k, v), tuple(synthetic.perturbed(x, 0.01, seed=200 + i) for i, x in enumerate((q, k, v)))]
    prev = [tuple(synthetic.perturbed(x, 0.01, seed=100 + 10 * b + i) for i, x in enumerate(clean[b]))
            for b in range(2)]
    attn = EchoSparseAttention(density=0.1, dense_steps=2, dense_layers=())
    for step in range(2):
        for b in range(2):
            attn(*(x[None] for x in prev[b]), step, b, 1)
    log("full-size sparse step: branch 0 and branch 1 of the first sparse step")
    attn(*(x[None] for x in clean[0]), 2, 0, 1)
    st = attn._states[1]
    prior1 = st.offset(1).clone()
    out1 = attn(*(x[None] for x in clean[1]), 2, 1, 1)[0]
    attn._flush_selection()
    torch.cuda.synchronize()
    buf, ps = attn._buffers, attn._plan_scratch
    b1 = dict(out=f32(out1), lse=f32(st.offset(1)), prior=prior1.cpu().numpy(), flags=buf.flags1.cpu().numpy(),
              k_mean=f32(buf.k_mean1), v_mean=f32(buf.v_mean1), k_rep=f32(buf.reps.k), v_rep=f32(buf.reps.v),
              log_counts=f32(buf.reps.log_counts))
    lists = dict(keep=ps.keep.cpu().numpy(), counts=ps.counts.cpu().numpy(), blocks=ps.blocks.cpu().numpy(),
                 means=ps.means.cpu().numpy(), mean_counts=ps.mean_counts.cpu().numpy(),
                 refine=ps.refine.cpu().numpy(), refine_counts=ps.refine_counts.cpu().numpy())
    # branch 0's block means and representatives, rebuilt for the direct launches below
    reps = attn.K.Representatives(q.shape[0], H, D, dev)
    km0, vm0 = torch.empty_like(buf.k_mean), torch.empty_like(buf.v_mean)
    reps.build(q, k, v, km0, vm0)
    torch.cuda.synchronize()
    return dict(attn=attn, clean=clean, b1=b1, lists=lists, km0=km0, vm0=vm0, reps0=reps)


def tile_inputs(x, t, h, L):
    """One head of x (L, H, D) as float32 with tile t's rows moved to rows 0.. (the oracle's tile 0)."""
    xh = f32(x[:, h:h + 1])
    r0, r1 = t * BM, min(t * BM + BM, L)
    xh[:r1 - r0] = xh[r0:r1]
    return xh


def oracle_fixed(q, k, v, lists, t, h, prior_col, comp_src, write_mass=False):
    """Oracle of the fixed-offset sparse step of pair (t, h): (O rows, LSE rows, flag, mass of the tile or None)."""
    L = q.shape[0]
    nq = ref.cdiv(L, BM)
    r0, r1 = t * BM, min(t * BM + BM, L)
    pr = np.full((nq * BM, 1), 1e30, np.float32)  # rows past the tile's valid rows hold the "no row" marker
    pr[:r1 - r0, 0] = prior_col[r0:r1]
    comp = dict(k_mean=comp_src["k_mean"][:, h:h + 1], v_mean=comp_src["v_mean"][:, h:h + 1],
                means=lists["means"][t:t + 1, h:h + 1], mean_counts=lists["mean_counts"][t:t + 1, h:h + 1],
                refine=lists["refine"][t:t + 1, h:h + 1], refine_counts=lists["refine_counts"][t:t + 1, h:h + 1],
                k_rep=comp_src["k_rep"][h:h + 1], v_rep=comp_src["v_rep"][h:h + 1],
                log_counts=comp_src["log_counts"][h:h + 1])
    ro, rl, _, rm = ref.fixed_offset_attention(tile_inputs(q, t, h, L), f32(k[:, h:h + 1]), f32(v[:, h:h + 1]),
                                                lists["counts"][t:t + 1, h:h + 1], lists["blocks"][t:t + 1, h:h + 1],
                                                pr, comp=comp, write_mass=write_mass, tiles=1)
    n = r1 - r0
    assert np.isfinite(rl[:BM]).all()   # (rows of the tiles past the first are not evaluated)
    # the kernel flags a tile from its valid rows only: log2 of a row total = LSE - prior outside [-60, 60]
    lg = rl[:n, 0] - pr[:n, 0].astype(np.float64)
    return ro[:n, 0], rl[:n, 0], int(np.any(~(np.abs(lg) <= 60.0))), rm


def oracle_fallback(q, k, v, lists, t, h, lse0_col, k_mean, v_mean):
    """Oracle of the flagged pair (t, h): online softmax over the tile's list, then the block-mean compensation of
    its keep == 0 blocks at the new LSE (O rows, LSE rows)."""
    L = q.shape[0]
    nq = ref.cdiv(L, BM)
    r0, r1 = t * BM, min(t * BM + BM, L)
    n = r1 - r0
    qh = tile_inputs(q, t, h, L)
    out = np.zeros((L, 1, D))
    lse = np.full((nq * BM, 1), 1e30)
    lse[:n, 0] = lse0_col[r0:r1]
    flags = np.zeros((nq, 1), np.int32)
    flags[0, 0] = 1
    kh, vh = f32(k[:, h:h + 1]), f32(v[:, h:h + 1])
    ref.exact_fallback(qh, kh, vh, out, lists["counts"][t:t + 1, h:h + 1], lists["blocks"][t:t + 1, h:h + 1], lse,
                       flags)
    ref.compensate_fallback(qh, k_mean[:, h:h + 1], v_mean[:, h:h + 1], lists["keep"][h:h + 1, t:t + 1], lse, out,
                            flags)
    return out[:n, 0], lse[:n, 0]


def test_sparse_step_full_shape_branch0(wan):
    attn, lists = wan["attn"], wan["lists"]
    q, k, v = wan["clean"][0]
    K, ps, st = attn.K, attn._plan_scratch, attn._states[1]
    L = q.shape[0]
    nq, nb = ref.cdiv(L, BM), ref.cdiv(L, 64)
    assert (L, nq, nb) == (75600, 591, 1182)
    out = torch.empty_like(q)
    lse = torch.empty_like(st.offset(0))
    flags = torch.empty(nq, H, device=q.device, dtype=torch.int32)
    mass = torch.zeros(H, nq, nb, device=q.device)
    R = wan["reps0"]
    log("full-size sparse step: branch-0 kernel")
    K.sparse_attention(q, k, v, wan["km0"], wan["vm0"], ps.means, ps.mean_counts, out, ps.counts, ps.blocks,
                       st.offset(0), lse, flags, ps.refine, ps.refine_counts, R.k, R.v, R.log_counts, mass=mass)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    c = lists
    assert c["counts"].mean() > 100 and c["mean_counts"].mean() > 100 and c["refine_counts"].mean() > 100
    prior = st.offset(0).cpu().numpy()
    comp = dict(k_mean=f32(wan["km0"]), v_mean=f32(wan["vm0"]), k_rep=f32(R.k), v_rep=f32(R.v),
                log_counts=f32(R.log_counts))
    go, gl, gf, gm = f32(out), f32(lse), flags.cpu().numpy(), f32(mass)
    for t, h in PAIRS:
        log("full-size branch 0: oracle tile", t, "head", h)
        ro, rl, rf, rm = oracle_fixed(q, k, v, lists, t, h, prior[:, h], comp, write_mass=True)
        r0, r1 = t * BM, min(t * BM + BM, L)
        check_close(f"O t{t} h{h}", go[r0:r1, h], ro)
        check_close(f"LSE t{t} h{h}", gl[r0:r1, h], rl)
        assert gf[t, h] == rf
        ex = c["blocks"][t, h, :c["counts"][t, h]]
        check_close(f"mass t{t} h{h}", gm[h, t, ex], rm[0, 0, ex], max_abs=2e-2 * max(1.0, float(np.abs(rm).max())))
        if r1 - r0 < BM:
            assert (gl[r1:r0 + BM, h] == 1e30).all()


def test_sparse_step_full_shape_branch1_reuses_the_plan(wan):
    """Branch 1's call in the pipeline: its output, LSE and flags for sampled pairs, with its own block means,
    representatives and prior over branch 0's lists."""
    b1, lists = wan["b1"], wan["lists"]
    q, k, v = wan["clean"][1]
    L = q.shape[0]
    assert np.isfinite(b1["out"]).all()
    for t, h in PAIRS_B1:
        log("full-size branch 1: oracle tile", t, "head", h)
        r0, r1 = t * BM, min(t * BM + BM, L)
        ro, rl, rf, _ = oracle_fixed(q, k, v, lists, t, h, b1["prior"][:, h], b1)
        assert b1["flags"][t, h] == rf
        if rf:
            ro, rl = oracle_fallback(q, k, v, lists, t, h, rl, b1["k_mean"], b1["v_mean"])
        check_close(f"branch-1 O t{t} h{h}", b1["out"][r0:r1, h], ro)
        check_close(f"branch-1 LSE t{t} h{h}", b1["lse"][r0:r1, h], rl)


def test_forced_fallback_full_shape(wan):
    """offset + 200 (the reference's fallback test) makes every row total 2^-200 of its value, so every tile is
    flagged; the fallback then recomputes O and LSE over the tile's list and compensates with the block means of its
    skipped blocks."""
    attn, lists = wan["attn"], wan["lists"]
    q, k, v = wan["clean"][0]
    K, ps, st = attn.K, attn._plan_scratch, attn._states[1]
    L = q.shape[0]
    nq = ref.cdiv(L, BM)
    R = wan["reps0"]
    shifted = st.offset(0) + 200.0
    shifted[L:] = 1e30
    out = torch.empty_like(q)
    lse = torch.empty_like(shifted)
    flags = torch.zeros(nq, H, device=q.device, dtype=torch.int32)
    log("full-size forced fallback: kernels")
    K.sparse_attention(q, k, v, wan["km0"], wan["vm0"], ps.means, ps.mean_counts, out, ps.counts, ps.blocks,
                       shifted, lse, flags, ps.refine, ps.refine_counts, R.k, R.v, R.log_counts)
    K.exact_fallback(q, k, v, out, ps.counts, ps.blocks, lse, flags)
    K.compensate_fallback(q, wan["km0"], wan["vm0"], ps.keep, lse, out, flags)
    torch.cuda.synchronize()
    assert (flags == 1).all(), "every tile must fall back"
    go, gl = f32(out), f32(lse)
    km, vm = f32(wan["km0"]), f32(wan["vm0"])
    for t, h in PAIRS_FALLBACK:
        log("full-size forced fallback: oracle tile", t, "head", h)
        r0, r1 = t * BM, min(t * BM + BM, L)
        ro, rl = oracle_fallback(q, k, v, lists, t, h, np.zeros(L), km, vm)
        check_close(f"fallback O t{t} h{h}", go[r0:r1, h], ro)
        check_close(f"fallback LSE t{t} h{h}", gl[r0:r1, h], rl)
