"""Bit-exact parity of the plan kernels (es_select_blocks, es_pack_plan, es_rebuild_plan) with the CPU oracle at
every block-count template the selection dispatches: select_kernel<E> with E = next_pow2(nb) / 256 in {1, 2, 4, 8,
16} (nb = 200, 300, 600, 1182 = the Wan2.1-14B map, 3000), i.e. 8 to 128 words of skip bits per (tile, head).

Two maps per size: a smooth Morton-like map (probability decaying away from the tile's own blocks, the shape real
maps have) with the reference's 10 % budget, and an adversarial one with heavy ties (values in quarter steps), NaN
entries, fell-back tiles and a sink. Reference semantics: echosparse/kernels/triton_ops.py:43-119 (selection),
sm120.py:258-305 (pack / rebuild)."""
import sys

import numpy as np
import pytest
import torch

from oracle import echosparse_ref as ref

pytestmark = pytest.mark.gpu

H = 2
SIZES = [200, 300, 600, 1182, 3000]


def K():
    from self_trainable_or_free_attn_amd.kernels import gfx950
    return gfx950


def _maps(nb, case, seed):
    """(L, mass, keep_prev, scale_exact, scale_skip, flags, sink) for a map of nb blocks (the last block holds 20
    tokens, so every size has a ragged tail)."""
    g = np.random.default_rng(seed)
    L = (nb - 1) * 64 + 20
    nq = ref.cdiv(L, 128)
    j = np.arange(nb)[None, None, :]
    t = np.arange(nq)[None, :, None]
    if case == "smooth":
        width = g.uniform(8.0, 64.0, size=(H, 1, 1))
        mass = np.exp(-np.abs(j - 2 * t) / width) * g.uniform(0.9, 1.1, size=(H, nq, nb))
        mass = (mass / mass.sum(-1, keepdims=True)).astype(np.float32)
        keep_prev = (g.random((H, nq, nb)) < 0.1).astype(np.uint8)
        se = g.uniform(0.5, 2.0, size=(H, nq)).astype(np.float32)
        ss = g.uniform(0.5, 2.0, size=(H, nq)).astype(np.float32)
        flags = np.zeros((nq, H), np.int32)
        sink = 1 << 30
    else:
        mass = g.integers(0, 5, size=(H, nq, nb)).astype(np.float32) / 4
        mass[g.random(mass.shape) < 0.05] = np.nan
        keep_prev = (g.random((H, nq, nb)) < 0.2).astype(np.uint8)
        se = np.ones((H, nq), np.float32)
        ss = np.full((H, nq), 0.5, np.float32)
        flags = np.zeros((nq, H), np.int32)
        flags[::3, 0] = 1
        flags[1::5, 1] = 1
        sink = nb - 20
    return L, mass, keep_prev, se, ss, flags, sink


@pytest.mark.parametrize("nb", SIZES)
@pytest.mark.parametrize("case", ["smooth", "ties"])
def test_select_pack_rebuild_bit_exact_at_size(nb, case, dev):
    top, refined = ref.budget(0.1, nb)
    rr, rc = _check(nb, case, top, refined, dev)
    # the case must exercise what it claims: a non-trivial refine list, and (ties) kept sets beyond the budget
    assert (rr < nb).any()
    if case == "ties":
        assert (rc > top).any()


# budgets at the ends of the K-th largest search: nothing (K = 0: the threshold is +inf, only forced and infinite
# entries are kept), one block, every block (K = nb: at most nb values, the threshold falls to the smallest), and
# a refine budget as large as the block count
EDGE_BUDGETS = {"none": lambda nb: (0, 0), "one": lambda nb: (1, 1), "all": lambda nb: (nb, 0),
                "refine_all": lambda nb: (0, nb)}


@pytest.mark.parametrize("nb", [300, 1182])
@pytest.mark.parametrize("case", ["smooth", "ties"])
@pytest.mark.parametrize("budget", sorted(EDGE_BUDGETS))
def test_select_bit_exact_at_edge_budgets(nb, case, budget, dev):
    top, refined = EDGE_BUDGETS[budget](nb)
    _check(nb, case, top, refined, dev)


def _check(nb, case, top, refined, dev):
    """select_blocks, pack_plan and rebuild_plan on one map against the oracle, byte for byte; returns the oracle's
    refine lists and counts."""
    L, mass, keep_prev, se, ss, flags, sink = _maps(nb, case, seed=nb + (case == "ties"))
    nq = ref.cdiv(L, 128)
    rw, words = -(-refined // 32) * 32, ref.plan_words(nb)
    print(f"[plans] nb={nb} case={case} L={L} E={max(1, ref.next_pow2(nb) // 256)} top={top} refined={refined}",
          flush=True)
    sys.stdout.flush()
    rk, rc, rb, rr, rs = ref.select_blocks(mass, keep_prev, se, ss, flags, top, refined, L, rw, words, sink=sink)

    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    keep = torch.full((H, nq, nb), 7, device=dev, dtype=torch.uint8)
    counts = torch.full((nq, H), 7, device=dev, dtype=torch.int32)
    blocks = torch.zeros(nq, H, nb, device=dev, dtype=torch.int32)
    skip = torch.full((H, nq, words), -1, device=dev, dtype=torch.int32)
    refine = torch.full((nq, H, rw), 7, device=dev, dtype=torch.int32)
    K().select_blocks(t(mass), t(keep_prev), t(se), t(ss), keep, counts, blocks, t(flags), skip, refine, top, refined,
                      L, sink=sink)
    torch.cuda.synchronize()
    assert np.array_equal(keep.cpu().numpy(), rk), "keep"
    assert np.array_equal(counts.cpu().numpy(), rc), "counts"
    used = np.arange(nb)[None, None, :] < rc[..., None]
    assert np.array_equal(blocks.cpu().numpy()[used], rb[used]), "blocks"
    assert np.array_equal(refine.cpu().numpy(), rr), "refine"
    assert np.array_equal(skip.cpu().numpy(), rs), "skip bits"

    exact = torch.full((H, nq, words), 5, device=dev, dtype=torch.int32)
    K().pack_plan(keep, exact)
    torch.cuda.synchronize()
    rex = ref.pack_plan(rk, words)
    assert np.array_equal(exact.cpu().numpy(), rex), "exact bits"

    lk, lc, lr, lrc, lmc = (torch.full(s, 7, device=dev, dtype=d) for s, d in
                            [((H, nq, nb), torch.uint8), ((nq, H), torch.int32), ((nq, H, rw), torch.int32),
                             ((nq, H), torch.int32), ((nq, H), torch.int32)])
    lb, lm = (torch.zeros(nq, H, nb, device=dev, dtype=torch.int32) for _ in range(2))
    K().rebuild_plan(exact, skip, lk, lc, lb, lr, lrc, lm, lmc)
    torch.cuda.synchronize()
    ok, oc, ob, orf, orc, om, omc = ref.rebuild_plan(rex, rs, nb, rw)
    assert np.array_equal(lk.cpu().numpy(), ok) and np.array_equal(ok, rk), "rebuilt keep"
    assert np.array_equal(lc.cpu().numpy(), oc) and np.array_equal(oc, rc), "rebuilt counts"
    used = np.arange(nb)[None, None, :] < oc[..., None]
    assert np.array_equal(lb.cpu().numpy()[used], ob[used]), "rebuilt blocks"
    assert np.array_equal(lr.cpu().numpy(), orf) and np.array_equal(orf, rr), "rebuilt refine"
    assert np.array_equal(lrc.cpu().numpy(), orc), "refine counts"
    assert np.array_equal(lmc.cpu().numpy(), omc), "mean counts"
    used = np.arange(nb)[None, None, :] < omc[..., None]
    assert np.array_equal(lm.cpu().numpy()[used], om[used]), "mean lists"
    return rr, rc
