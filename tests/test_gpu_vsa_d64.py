"""Parity of the VSA ops at head dim D = 64 (the C ABI stores rows with 128 columns and takes the logical D; the op
layer zero-pads and narrows) with the CPU oracle (oracle/vsa_ref.py): pooled means and selections bit for bit,
outputs and gradients at max-abs 2e-2 / rel-L2 1e-2.

Shapes: the reference's CPU configuration (B = 1, H = 2, N = 4096 = 64 blocks, D = 64, top-16 key blocks per query
block by mean-pooled score, reference tests/vsa_reference.py) with bf16 inputs, and NB = 10 with partial blocks for
the operators, split-KV and the three tiers."""
import sys

import numpy as np
import pytest
import torch

from helpers import bf16_max_abs, check_close, f32
from oracle import vsa_ref as ref

pytestmark = pytest.mark.gpu

D = 64
CNT = [64, 64, 37, 64, 1, 64, 64, 20, 64, 50]
NB = len(CNT)
L = NB * 64


def C():
    from self_trainable_or_free_attn_amd.vsa import _C
    return _C


def ops():
    from self_trainable_or_free_attn_amd.vsa import ops as o
    return o


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def tokens(seed, dev, shape, cnt):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    x = (x * torch.as_tensor(ref.token_valid(cnt, shape[2]))[None, None, :, None]).to(torch.bfloat16)
    return x, x.to(dev)


@pytest.fixture(scope="module")
def small(dev):
    out = [tokens(s, dev, (1, 2, L, D), CNT) for s in (1, 2, 3)]
    return dict(cpu=[o[0] for o in out], gpu=[o[1] for o in out],
                blk=torch.tensor(CNT, dtype=torch.int32, device=dev))


def test_c1_route_and_forward(dev):
    """The reference's CPU benchmark case at D = 64: top-16 of 64 key blocks per query block, O and LSE."""
    log("C1 D64 route_rows + fine forward")
    nb, n = 64, 4096
    cnt = [64] * nb
    x = [tokens(s, dev, (1, 2, n, D), cnt) for s in (0, 1, 2)]
    q, k, v = (t[1] for t in x)
    blk = torch.tensor(cnt, dtype=torch.int32, device=dev)
    _, _, qc, kc, _ = C().pool_fwd(q, k, v, blk, 32)
    assert qc.shape[-1] == D
    _, want_qc = ref.pool(f32(x[0][0]), cnt, 32)
    assert np.array_equal(f32(qc)[:, :, :nb], want_qc)
    scores = f32(C().block_scores(qc, kc, nb))
    want_s = ref.block_scores(f32(qc)[:, :, :nb], f32(kc)[:, :, :nb]).reshape(2, nb, nb)
    step = np.exp2(np.floor(np.log2(np.maximum(np.abs(want_s), 2.0 ** -100))) - 7)
    assert (np.abs(scores - want_s) <= step + 1e-30).all()
    sel = C().route_rows(qc, kc, nb, 16)
    mask = ref.row_topk_mask(scores.reshape(1, 2, nb, nb), 16)
    rp, ri = ref.csr_from_mask(mask)
    assert np.array_equal(sel[0].cpu().numpy(), rp) and np.array_equal(sel[1].cpu().numpy()[:ri.size], ri)
    o, lse = C().attn_fwd(q, k, v, sel[0], sel[1], blk)
    torch.cuda.synchronize()
    assert o.shape == q.shape
    wo, wl = ref.fine_attention(*(f32(t[0]) for t in x), cnt, mask)
    check_close("O", f32(o), wo)
    check_close("lse", f32(lse), wl)


@pytest.mark.parametrize("seed", [0, 1])
def test_fine_forward_backward(small, seed):
    log("D64 fine fwd/bwd seed", seed)
    q, k, v = (t.detach().clone().requires_grad_(True) for t in small["gpu"])
    g = np.random.default_rng(seed)
    m = g.random((1, 2, NB, NB)) < 0.4
    m[:, :, 0] = True
    m[:, :, 1] = False
    sel = ops().mask_to_selection(torch.as_tensor(m).to(q.device))
    o, lse = ops().fine_block_sparse_attention(q, k, v, small["blk"], sel)
    dout_c, dout = tokens(20 + seed, q.device, (1, 2, L, D), CNT)
    grads = torch.autograd.grad(o, (q, k, v), dout)
    torch.cuda.synchronize()
    wo, wl = ref.fine_attention(*(f32(x) for x in small["cpu"]), CNT, m)
    check_close("O", f32(o), wo)
    fin = np.isfinite(wl)
    assert np.array_equal(np.isfinite(f32(lse)), fin)
    check_close("lse", f32(lse)[fin], wl[fin])
    wg = ref.fine_backward(*(f32(x) for x in small["cpu"]), CNT, m, f32(dout_c))
    for name, a, w in zip(("dQ", "dK", "dV"), grads, wg):
        assert a.shape == q.shape
        check_close(name, f32(a), w)


def test_split_equals_unsplit(small):
    log("D64 split-KV")
    q, k, v = (t.detach().clone().requires_grad_(True) for t in small["gpu"])
    m = np.random.default_rng(3).random((1, 2, NB, NB)) < 0.8
    sel = ops().mask_to_selection(torch.as_tensor(m).to(q.device))
    dout = tokens(31, q.device, (1, 2, L, D), CNT)[1]
    o1, _ = ops().fine_block_sparse_attention(q, k, v, small["blk"], sel)
    g1 = torch.autograd.grad(o1, (q, k, v), dout)
    split = ops().SplitKV(chunk=3)
    o2, _ = ops().fine_block_sparse_attention(q, k, v, small["blk"], sel, split_kv=split)
    g2 = torch.autograd.grad(o2, (q, k, v), dout)
    assert ops().describe_split(q, sel, split)["fwd"]["info"]["split_rows"] > 0
    check_close("O split", f32(o2), f32(o1), max_abs=1e-2, rel=5e-3)
    for name, a, b in zip(("dQ", "dK", "dV"), g2, g1):
        check_close(name + " split", f32(a), f32(b), max_abs=1e-2, rel=5e-3)


@pytest.mark.parametrize("which", ["vsa", "vsa2"])
def test_operators(small, which):
    log("D64 operator", which)
    q, k, v = (x.detach().clone().requires_grad_(True) for x in small["gpu"])
    g = torch.Generator().manual_seed(60)
    if which == "vsa2":
        gate_c = torch.randn(1, 2, L, generator=g).to(torch.bfloat16)
        gate = gate_c.to(q.device).requires_grad_(True)
        o, sel = ops().vsa2_attention(q, k, v, gate, small["blk"], R=16, topk=3, return_selection=True)
        act, R = "tanh", 16
    else:
        gate_c = (torch.randn(1, 2, L, D, generator=g) * 0.5).to(torch.bfloat16)
        gate = gate_c.to(q.device).requires_grad_(True)
        o, sel = ops().vsa_attention(q, k, v, small["blk"], 4, weight=gate, return_selection=True)
        act, R = "identity", 32
    dout_c, dout = tokens(61, q.device, (1, 2, L, D), CNT)
    grads = torch.autograd.grad(o, (q, k, v, gate), dout)
    mask = sel.to_mask(NB).cpu().numpy()
    _, _, qc, kc, vc = C().pool_fwd(*small["gpu"], small["blk"], R)
    pooled = [f32(x)[:, :, :NB] for x in (qc, kc, vc)]
    leaves = [x.double().requires_grad_(True) for x in (*small["cpu"], gate_c)]
    want = ref.vsa_output(*leaves[:3], leaves[3], CNT, mask, act, pooled=pooled)
    wg = torch.autograd.grad(want, leaves, dout_c.double())
    assert o.shape == q.shape
    check_close(which + " O", f32(o), want.detach().numpy())
    for name, a, w in zip(("dQ", "dK", "dV", "dgate"), grads, wg):
        assert a.shape == w.shape
        check_close(which + " " + name, f32(a), w.numpy())


def test_three_tiers(small):
    log("D64 three tiers")
    from self_trainable_or_free_attn_amd.vsa import rep
    q, k, v = (t.detach().clone().requires_grad_(True) for t in small["gpu"])
    g = np.random.default_rng(5)
    a = g.random((1, 2, NB, NB)) < 0.15
    ab = a | (g.random((1, 2, NB, NB)) < 0.3)
    sa = ops().mask_to_selection(torch.as_tensor(a).to(q.device))
    sel = rep.TierSelection(sa.q2k_ptr, sa.q2k_idx, sa.k2q_ptr, sa.k2q_idx, rep.pack_bits(torch.as_tensor(a).to(q.device)),
                            rep.pack_bits(torch.as_tensor(ab).to(q.device))).with_tier_b()
    RM = 4
    o, _ = rep.rep_fine_attention(q, k, v, small["blk"], sel, mid_reps=RM, phases=7)
    dout_c, dout = tokens(40, q.device, (1, 2, L, D), CNT)
    grads = torch.autograd.grad(o, (q, k, v), dout)
    torch.cuda.synchronize()
    km, vm, kt, vt, _, _ = ref.rep_tables(f32(small["cpu"][1]), f32(small["cpu"][2]), CNT, RM)
    x = [t.double().requires_grad_(True) for t in small["cpu"]]
    wo, _ = ref.rep_fine_torch(*x, CNT, a, ab, RM, 7, tables=(km, vm, kt, vt))
    wg = torch.autograd.grad(wo, x, dout_c.double())
    check_close("O", f32(o), wo.detach().numpy())
    for name, gr, w in zip(("dQ", "dK", "dV"), grads, wg):
        check_close(name, f32(gr), w.numpy(), max_abs=bf16_max_abs(w.numpy()))
