"""The EchoSparse schedule end to end on the GPU (the reference's tests/test_attention.py and the state / rows tests
of tests/test_sm120.py, restated): density 1.0 equals dense attention, CFG branches share branch 0's selection,
a sparse step equals the explicit one-softmax formula, far-off offsets fall back to the exact result, `rows` skips
only unused tiles, and the persistent state keeps its size. References are fp32 torch on the same device."""
import math
import sys

import pytest
import torch

from helpers import structured_qkv

pytestmark = pytest.mark.gpu

L, H, D = 4152, 2, 128          # 65 kv blocks (the last has 56 tokens), 33 query tiles (the last has 56 rows)


def steps(n, seed=0, dev="cuda", shape=(L, H)):
    return [[x[None].to(dev) for x in s] for s in structured_qkv(shape[0], shape[1], D, seed=seed, steps=n)]


def dense(q, k, v):
    """fp32 torch attention on [1, L, H, D] tensors."""
    qt, kt, vt = (x[0].float().permute(1, 0, 2) for x in (q, k, v))
    o = torch.softmax(qt @ kt.transpose(1, 2) / math.sqrt(D), -1) @ vt
    return o.permute(1, 0, 2)[None]


def rel_err(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


def run(attn, inputs, branches=1, layer=1):
    outs = []
    for step, (q, k, v) in enumerate(inputs):
        for branch in range(branches):
            outs.append(attn(q, k, v, step, branch, layer=layer))
    attn._flush_selection()       # a deferred selection is enqueued now,
    torch.cuda.synchronize()      # and settled (it runs on a side stream) before any state is read
    return outs


def call_with_selection(attn, q, k, v, step, branch=0, layer=1):
    """One sparse call; returns its output and the block selection it used (counts, blocks, refine list)."""
    attn._flush_selection()
    torch.cuda.synchronize()
    st = attn._states[layer]
    exact, skip = (x.clone() for x in st.plan(st.pending[0] if branch == 0 else st.current[0]))
    out = attn(q, k, v, step, branch, layer=layer)
    torch.cuda.synchronize()
    Hh, nq, _ = exact.shape
    nb = -(-q.shape[1] // 64)
    keep = torch.empty(Hh, nq, nb, device="cuda", dtype=torch.uint8)
    counts = torch.empty(nq, Hh, device="cuda", dtype=torch.int32)
    blocks = torch.zeros(nq, Hh, nb, device="cuda", dtype=torch.int32)
    refine = torch.empty_like(attn._plan_scratch.refine)
    lists = torch.empty_like(counts), torch.empty_like(blocks), torch.empty_like(counts)
    attn.K.rebuild_plan(exact, skip, keep, counts, blocks, refine, *lists)
    return out, (counts, blocks, refine)


def check_formula(out, qkv, selection, buf, branch=0):
    """Exact tokens of the listed blocks, block means of the other skipped blocks and four representatives of each
    refined block, all in one softmax (reference tests/test_attention.py:72-100). The block means are the branch's
    own (branch 0 keeps its set for its selection on the plan stream)."""
    out = out[0].float()
    q, k, v = (x[0].float() for x in qkv)
    L, H = q.shape[0], q.shape[1]
    counts, blocks, refine = selection
    k_mean, v_mean = (buf.k_mean, buf.v_mean) if branch == 0 else (buf.k_mean1, buf.v_mean1)
    nb = k_mean.shape[0]
    block_len = torch.full((nb,), 64.0, device="cuda")
    block_len[-1] = L - 64 * (nb - 1)
    nq = -(-L // 128)
    for h in range(H):
        for t in sorted({0, 7, nq // 2, nq - 1}):
            exact = blocks[t, h, :counts[t, h]].tolist()
            refined = [b for b in refine[t, h].tolist() if b < nb]
            means = sorted(set(range(nb)) - set(exact) - set(refined))
            rows = torch.arange(128 * t, min(128 * t + 128, L), 9, device="cuda")
            keys, vals, bias = [], [], []
            for b in exact:
                tok = torch.arange(64 * b, min(64 * b + 64, L), device="cuda")
                keys.append(k[tok, h]); vals.append(v[tok, h]); bias.append(torch.zeros(len(tok), device="cuda"))
            keys.append(k_mean[means, h].float()); vals.append(v_mean[means, h].float())
            bias.append(block_len[means].log())
            for b in refined:
                sl = slice(4 * b, 4 * b + 4)
                keys.append(buf.reps.k[h, sl].float()); vals.append(buf.reps.v[h, sl].float())
                bias.append(buf.reps.log_counts[h, sl] * math.log(2))
            logits = q[rows, h] @ torch.cat(keys).T / math.sqrt(D) + torch.cat(bias)
            ref = torch.softmax(logits, -1) @ torch.cat(vals)
            assert rel_err(out[rows, h], ref) < 1e-2, (h, t)


def new_attention(**kw):
    from self_trainable_or_free_attn_amd import EchoSparseAttention
    return EchoSparseAttention(dense_steps=2, dense_layers=(), **kw)


def test_full_density_matches_dense():
    inputs = steps(4)
    outs = run(new_attention(density=1.0), inputs)
    for (q, k, v), out in zip(inputs, outs):
        assert rel_err(out, dense(q, k, v)) < 1e-2


def test_cfg_branches_share_selection():
    inputs = steps(4)
    outs = run(new_attention(density=1.0), inputs, branches=2)
    for i, (q, k, v) in enumerate(inputs):
        ref = dense(q, k, v)
        assert rel_err(outs[2 * i], ref) < 1e-2 and rel_err(outs[2 * i + 1], ref) < 1e-2


def test_sparse_step_matches_formula():
    inputs = steps(3)
    attn = new_attention(density=0.1)
    run(attn, inputs[:2])
    out, selection = call_with_selection(attn, *inputs[2], 2)
    check_formula(out, inputs[2], selection, attn._buffers)


@pytest.mark.parametrize("shape", [(4097, 1), (4160, 2), (8191, 3)])
def test_sparse_step_matches_formula_at_edge_shapes(shape):
    """A last kv block of one token (its mean is that token, its log2 count 0, its representatives one point), a
    length that fills its last kv block but only half of its last query tile, and 128 kv blocks with a 63-token
    tail and a 127-row last tile, at 1 and 3 heads."""
    print("edge shape", shape, flush=True)
    inputs = steps(3, seed=3, shape=shape)
    attn = new_attention(density=0.1)
    run(attn, inputs[:2])
    out, selection = call_with_selection(attn, *inputs[2], 2)
    check_formula(out, inputs[2], selection, attn._buffers)


def test_second_cfg_branch_matches_formula():
    """The unconditional branch uses the conditional branch's block selection with its own inputs and offsets."""
    cond, uncond = steps(3, seed=1), steps(3, seed=2)
    attn = new_attention(density=0.1)
    for step in range(2):
        attn(*cond[step], step, 0, layer=1)
        attn(*uncond[step], step, 1, layer=1)
    _, first = call_with_selection(attn, *cond[2], 2, branch=0)
    out, second = call_with_selection(attn, *uncond[2], 2, branch=1)
    assert all(torch.equal(a, b) for a, b in zip(first, second))
    check_formula(out, uncond[2], second, attn._buffers, branch=1)


def test_fallback_tiles():
    """A far-off offset flags every tile; the online-softmax fallback must give the same result."""
    inputs = steps(4)
    attn = new_attention(density=1.0)
    run(attn, inputs[:3])
    attn._states[1].offset(0)[:L] += 200.0
    q, k, v = inputs[3]
    out = attn(q, k, v, 3, 0, layer=1)
    assert rel_err(out, dense(q, k, v)) < 1e-2


def test_sparse_fallback_compensates():
    """Sparse density with every tile flagged: online softmax over the listed blocks plus block-mean compensation
    of every keep == 0 block at the new LSE (reference triton_ops.py:251-295), against the same formula in torch."""
    inputs = steps(4)
    attn = new_attention(density=0.1)
    run(attn, inputs[:3])
    st = attn._states[1]
    exact, skip = (x.clone() for x in st.plan(st.pending[0]))
    st.offset(0)[:L] += 200.0
    q, k, v = inputs[3]
    out = attn(q, k, v, 3, 0, layer=1)[0].float()
    nb = -(-L // 64)
    bits = (exact.permute(1, 0, 2)[..., :, None] >> torch.arange(32, device="cuda")) & 1
    keep = bits.flatten(-2)[..., :nb].bool()                 # (nq, H, nb)
    buf = attn._buffers
    blen = torch.full((nb,), 64.0, device="cuda")
    blen[-1] = L - 64 * (nb - 1)
    qf, kf, vf = (x[0].float() for x in (q, k, v))
    for h in range(H):
        for t in (2, 32):
            rows = torch.arange(128 * t, min(128 * t + 128, L), device="cuda")
            ex = keep[t, h].nonzero().flatten().tolist()
            tok = torch.cat([torch.arange(64 * b, min(64 * b + 64, L), device="cuda") for b in ex])
            sk = (~keep[t, h]).nonzero().flatten()
            keys = torch.cat([kf[tok, h], buf.k_mean[sk, h].float()])
            vals = torch.cat([vf[tok, h], buf.v_mean[sk, h].float()])
            bias = torch.cat([torch.zeros(len(tok), device="cuda"), blen[sk].log()])
            ref = torch.softmax(qf[rows, h] @ keys.T / math.sqrt(D) + bias, -1) @ vals
            assert rel_err(out[rows, h], ref) < 1e-2, (h, t)


def test_rows_skip_only_unused_tiles():
    """`rows`: tiles past the used rows are not computed; their output is zero, their LSE the offset, their flag
    0 (reference tests/test_sm120.py:97-106)."""
    from self_trainable_or_free_attn_amd.kernels import gfx950 as K
    inputs = steps(3)
    attn = new_attention(density=0.1)
    run(attn, inputs[:2])
    q, k, v = (x[0] for x in inputs[2])
    st, ps, buf = attn._states[1], None, attn._buffers
    exact, skip = st.plan(st.pending[0])
    attn(*inputs[2], 2, 0, layer=1)          # builds scratch and representatives for this shape
    attn._flush_selection()
    torch.cuda.synchronize()
    ps = attn._plan_scratch
    K.rebuild_plan(exact, skip, ps.keep, ps.counts, ps.blocks, ps.refine, ps.refine_counts, ps.means,
                   ps.mean_counts)
    offset = st.offset(0).clone()

    def run_kernel(rows):
        out, lse = torch.full_like(q, 7.0), torch.full_like(offset, 7.0)
        flags = torch.full(buf.flags.shape, 7, device="cuda", dtype=torch.int32)
        mass = torch.zeros_like(ps.mass)
        K.sparse_attention(q, k, v, buf.k_mean, buf.v_mean, ps.means, ps.mean_counts, out, ps.counts, ps.blocks,
                           offset, lse, flags, ps.refine, ps.refine_counts, buf.reps.k, buf.reps.v,
                           buf.reps.log_counts, mass=mass, rows=rows)
        return out, lse, flags, mass

    same = lambda a, b: torch.equal(a.view(torch.uint8), b.view(torch.uint8))
    full = run_kernel(L)
    part = run_kernel(4000)                   # 32 tiles; tile 31 holds rows 3968-4095 and is computed whole
    assert same(part[0][:4096], full[0][:4096]) and same(part[1][:4096], full[1][:4096])
    assert same(part[2][:32], full[2][:32]) and same(part[3][:, :32], full[3][:, :32])
    assert part[0][4096:].abs().max() == 0 and same(part[1][4096:], offset[4096:])
    assert (part[2][32:] == 0).all()


def test_deterministic_rerun():
    """The same inputs give byte-identical outputs and state (fixed-order reductions, no atomics)."""
    def once():
        inputs = steps(3)
        attn = new_attention(density=0.1)
        outs = run(attn, inputs)
        return outs[-1], attn._states[1].offset(0).clone(), [x.clone() for x in attn._states[1].plan(0)]
    a, b = once(), once()
    assert torch.equal(a[0].view(torch.int16), b[0].view(torch.int16)) and torch.equal(a[1], b[1])
    assert all(torch.equal(x, y) for x, y in zip(a[2], b[2]))


def persistent_bytes(st):
    return sum(x.numel() * x.element_size() for x in [*st.offsets.values(), *(t for p in st.plans for t in p)])


def run_steps(attn, n, branches, sink=None):
    data = [steps(n, seed=3 + b) for b in range(branches)]
    for video in range(2):
        attn.reset()
        for step in range(n):
            for branch in range(branches):
                attn(*data[branch][step], step, branch, 1, sink=sink)
    torch.cuda.synchronize()
    return attn._states[1]


def test_plans_with_cfg():
    """Wan2.1 form: two CFG branches, the second reusing the first's plan; two plans per layer"""
    st = run_steps(new_attention(density=0.1), 6, branches=2)
    nq, words = -(-L // 128), st.words
    assert sorted(st.offsets) == [0, 1] and st.ready == {0, 1} and len(st.plans) == 2 and st.pending[1] == 6
    assert persistent_bytes(st) == 2 * nq * 128 * H * 4 + 4 * H * nq * words * 4


def test_plans_single_branch():
    """HunyuanVideo form: one branch, a text sink at the end; one plan per layer, rewritten in place"""
    st = run_steps(new_attention(density=0.1), 6, branches=1, sink=4096 // 64)
    nq, words = -(-L // 128), st.words
    assert sorted(st.offsets) == [0] and len(st.plans) == 1 and st.pending == (0, 6)
    assert persistent_bytes(st) == nq * 128 * H * 4 + 2 * H * nq * words * 4
