"""The sparse step at the full Wan2.1-14B shape (L = 75 600 = 1182 kv blocks, 591 query tiles with an 80-row tail
tile, H = 40, D = 128, density 0.10), through the production pipeline (two dense steps, then sparse steps with
the kernel-built plan, block means and representatives), checked against the CPU oracle on sampled (tile, head)
pairs: the oracle evaluates exactly the same column lists, so the check covers 32-bit addressing over the full
tensors, long lists through the staged list ring, the tail tile and the mass map at full size, at max-abs 2e-2 /
rel-L2 1e-2 (mass: 2e-2 of its largest value)."""
import sys

import numpy as np
import pytest
import torch

from helpers import check_close, f32
from oracle import echosparse_ref as ref

pytestmark = pytest.mark.gpu

GRID = (21, 45, 80)
H, D, BM = 40, 128, 128
PAIRS = [(0, 0), (295, 17), (590, 39), (123, 5)]  # (query tile, head); tile 590 is the 80-row tail


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_sparse_step_full_shape_sampled_tiles(dev):
    from self_trainable_or_free_attn_amd import EchoSparseAttention, synthetic
    log("full-size sparse step: building Wan-shaped inputs")
    q, k, v, _ = synthetic.fourier_qkv(GRID, H, D, seed=11, device=dev)
    prev = [synthetic.perturbed(x, 0.01, seed=100 + i) for i, x in enumerate((q, k, v))]
    attn = EchoSparseAttention(density=0.1, dense_steps=2, dense_layers=())
    for step in range(2):
        attn(prev[0][None], prev[1][None], prev[2][None], step, 0, 1)
    attn(q[None], k[None], v[None], 2, 0, 1)
    attn._flush_selection()
    torch.cuda.synchronize()
    K, ps, buf, st = attn.K, attn._plan_scratch, attn._buffers, attn._states[1]
    L = q.shape[0]
    nq, nb = ref.cdiv(L, BM), ref.cdiv(L, 64)
    assert (L, nq, nb) == (75600, 591, 1182)
    out = torch.empty_like(q)
    lse = torch.empty_like(st.offset(0))
    flags = buf.flags.clone()
    mass = torch.zeros_like(ps.mass)
    log("full-size sparse step: kernel")
    K.sparse_attention(q, k, v, buf.k_mean, buf.v_mean, ps.means, ps.mean_counts, out, ps.counts, ps.blocks,
                       st.offset(0), lse, flags, ps.refine, ps.refine_counts, buf.reps.k, buf.reps.v,
                       buf.reps.log_counts, mass=mass)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    counts, blocks = ps.counts.cpu().numpy(), ps.blocks.cpu().numpy()
    means, mc = ps.means.cpu().numpy(), ps.mean_counts.cpu().numpy()
    refine, rc = ps.refine.cpu().numpy(), ps.refine_counts.cpu().numpy()
    assert counts.mean() > 100 and mc.mean() > 100 and rc.mean() > 100  # long streams of every column kind
    prior = st.offset(0).cpu().numpy()
    km, vm = f32(buf.k_mean), f32(buf.v_mean)
    kr, vr, lc = f32(buf.reps.k), f32(buf.reps.v), f32(buf.reps.log_counts)
    go, gl, gf, gm = f32(out), f32(lse), flags.cpu().numpy(), f32(mass)
    for t, h in PAIRS:
        log("full-size sparse step: oracle tile", t, "head", h)
        r0, r1 = t * BM, min(t * BM + BM, L)
        # the oracle's tile 0 = this tile: its query rows and prior moved to rows 0.., one head, real L
        qh = f32(q[:, h:h + 1])
        qh[:r1 - r0] = qh[r0:r1]
        pr = np.full((nq * BM, 1), np.inf, np.float32)  # rows past the tile's valid rows: P = 0
        pr[:r1 - r0, 0] = prior[r0:r1, h]
        comp = dict(k_mean=km[:, h:h + 1], v_mean=vm[:, h:h + 1], means=means[t:t + 1, h:h + 1],
                    mean_counts=mc[t:t + 1, h:h + 1], refine=refine[t:t + 1, h:h + 1],
                    refine_counts=rc[t:t + 1, h:h + 1], k_rep=kr[h:h + 1], v_rep=vr[h:h + 1],
                    log_counts=lc[h:h + 1])
        ro, rl, _, rm = ref.fixed_offset_attention(qh, f32(k[:, h:h + 1]), f32(v[:, h:h + 1]),
                                                    counts[t:t + 1, h:h + 1], blocks[t:t + 1, h:h + 1], pr,
                                                    comp=comp, write_mass=True, tiles=1)
        n = r1 - r0
        check_close(f"O t{t} h{h}", go[r0:r1, h], ro[:n, 0])
        check_close(f"LSE t{t} h{h}", gl[r0:r1, h], rl[:n, 0])
        lg = rl[:n, 0] - pr[:n, 0]  # log2 of the row totals over the tile's valid rows
        assert gf[t, h] == int(np.any(~(np.abs(lg) <= 60.0)))
        ex = blocks[t, h, :counts[t, h]]
        check_close(f"mass t{t} h{h}", gm[h, t, ex], rm[0, 0, ex], max_abs=2e-2 * max(1.0, float(np.abs(rm).max())))
        if r1 - r0 < BM:
            assert (gl[r1:r0 + BM, h] == 1e30).all()
