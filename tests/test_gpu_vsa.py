"""Parity of the VSA / VSA2 kernels (include/vsa_hip.h) with the CPU oracle (oracle/vsa_ref.py), through the
native op set (self_trainable_or_free_attn_amd.vsa._C, thin ctypes calls) and the operators.

Integer work (pooled values restating the kernel's float32 order, selections, CSR lists, split plans) is compared
bit for bit; floating-point outputs at max-abs 2e-2 and rel-L2 1e-2 (gradients: the same bounds). Shapes: NB = 10
(L = 640) with partial blocks (the reference's tests use blk_cnt patterns like [64, 1, 64, 37, 20]), B = 1, H = 2,
D = 128, plus router edge cases (NB not a multiple of 32, K = 0, K = NB, ties, -0 / +0)."""
import math
import sys

import numpy as np
import pytest
import torch

from helpers import bf16_max_abs, check_close, f32
from oracle import vsa_ref as ref

pytestmark = pytest.mark.gpu

B, H, D = 1, 2, 128
CNT = [64, 64, 37, 64, 1, 64, 64, 20, 64, 50]
NB = len(CNT)
L = NB * 64


def C():
    from self_trainable_or_free_attn_amd.vsa import _C
    return _C


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def tokens(seed, dev, shape=(B, H, L, D), cnt=CNT, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g) * scale
    valid = torch.as_tensor(ref.token_valid(cnt, shape[2]))[None, None, :, None]
    x = (x * valid).to(torch.bfloat16)
    return x, x.to(dev)


@pytest.fixture(scope="module")
def qkv(dev):
    out = [tokens(s, dev) for s in (1, 2, 3)]
    blk = torch.tensor(CNT, dtype=torch.int32, device=dev)
    return dict(cpu=[o[0] for o in out], gpu=[o[1] for o in out], blk=blk)


def random_mask(seed, nb=NB, density=0.4):
    g = np.random.default_rng(seed)
    m = g.random((B, H, nb, nb)) < density
    m[:, :, 0, :] = True          # a full row
    m[:, :, :, 2] |= True         # a column with a partial block
    m[:, :, 1, :] = False         # an empty row
    return m


def selection_of(mask, dev):
    from self_trainable_or_free_attn_amd.vsa import ops
    return ops.mask_to_selection(torch.as_tensor(mask).to(dev))


# --------------------------------------------------------------------------- pooling
@pytest.mark.parametrize("R", [4, 8, 16, 32])
def test_pool_bit_exact(qkv, R):
    log("pool R", R)
    q, k, v = qkv["gpu"]
    qr, kr, qc, kc, vc = C().pool_fwd(q, k, v, qkv["blk"], R)
    torch.cuda.synchronize()
    G = 64 // R
    for name, x, g_out, b_out in (("q", qkv["cpu"][0], qr, qc), ("k", qkv["cpu"][1], kr, kc)):
        grp, blk = ref.pool(f32(x), CNT, R)
        assert np.array_equal(f32(g_out)[:, :, :NB * G], grp), f"{name} group means differ"
        assert np.array_equal(f32(b_out)[:, :, :NB], blk), f"{name} block means differ"
        assert (f32(g_out)[:, :, NB * G:] == 0).all() and (f32(b_out)[:, :, NB:] == 0).all()
    _, vblk = ref.pool(f32(qkv["cpu"][2]), CNT, R)
    assert np.array_equal(f32(vc)[:, :, :NB], vblk)


def test_pool_never_reads_padding(dev):
    cnt = [64, 10, 33]
    x = torch.randn(1, 1, 192, 128)
    x[:, :, 64 + 10:128] = float("nan")
    x[:, :, 128 + 33:] = float("inf")
    xd = x.to(torch.bfloat16).to(dev)
    blk = torch.tensor(cnt, dtype=torch.int32, device=dev)
    qr, kr, qc, kc, vc = C().pool_fwd(xd, xd, xd, blk, 8)
    assert torch.isfinite(qr.float()).all() and torch.isfinite(qc.float()).all()


# --------------------------------------------------------------------------- original-VSA router
def _csr_to_mask(ptr, idx, nb):
    return ref.mask_from_csr(ptr.cpu().numpy(), idx.cpu().numpy(), nb)


def _check_csr(q2k_ptr, q2k_idx, k2q_ptr, k2q_idx, want, per_head):
    """CSR lists == the mask, rows ascending, bases bh * per_head, k2q = the transposed lists."""
    nb = want.shape[-1]
    qp, qi = q2k_ptr.cpu().numpy(), q2k_idx.cpu().numpy()
    kp, ki = k2q_ptr.cpu().numpy(), k2q_idx.cpu().numpy()
    rp, ri = ref.csr_from_mask(want)
    assert np.array_equal(qp, rp) and np.array_equal(qi[:ri.size], ri), "q2k lists differ"
    cp, ci = ref.csr_from_mask(np.swapaxes(want, -1, -2))
    assert np.array_equal(kp, cp) and np.array_equal(ki[:ci.size], ci), "k2q lists differ"
    BH = want.shape[0] * want.shape[1]
    assert np.array_equal(qp.reshape(BH, nb + 1)[:, 0], np.arange(BH) * per_head)


@pytest.mark.parametrize("K", [0, 1, 3, 7, 10])
def test_route_rows_bit_exact(qkv, K):
    log("route_rows K", K)
    q, k, _ = qkv["gpu"]
    _, _, qc, kc, _ = C().pool_fwd(q, k, k, qkv["blk"], 32)
    scores = C().block_scores(qc, kc, NB)
    got = C().route_rows(qc, kc, NB, K)
    torch.cuda.synchronize()
    # the score op: float64 dot rounded twice; the GPU's fp32 dot may land one bf16 step away on rare entries
    want_s = ref.block_scores(f32(qc)[:, :, :NB], f32(kc)[:, :, :NB]).reshape(B * H, NB, NB)
    gs = f32(scores)
    step = np.exp2(np.floor(np.log2(np.maximum(np.abs(want_s), 2.0 ** -100))) - 7)
    assert (np.abs(gs - want_s) <= step + 1e-30).all()
    assert (gs == want_s).mean() > 0.95
    # selection: bit-exact on the GPU's own scores
    want = ref.row_topk_mask(gs.reshape(B, H, NB, NB), K)
    _check_csr(*got, want, NB * K)


def test_row_topk_known_answers(dev):
    """Ties and -0 == +0 (reference tests/test_vsa.py:67-73), on the row top-K kernel with given scores."""
    s = torch.tensor([[0.5, 0.0, -0.0, 0.5, 0.25, 0.0]] * 6, dtype=torch.bfloat16).reshape(1, 6, 6).to(dev)
    for K, row in ((3, [0, 3, 4]), (4, [0, 1, 3, 4]), (5, [0, 1, 2, 3, 4]), (6, [0, 1, 2, 3, 4, 5]), (0, [])):
        out = [torch.empty(1, 1, 7, dtype=torch.int32, device=dev), torch.empty(max(6 * K, 1), dtype=torch.int32,
               device=dev), torch.empty(1, 1, 7, dtype=torch.int32, device=dev),
               torch.empty(max(6 * K, 1), dtype=torch.int32, device=dev)]
        C().row_topk_into(s, K, 0, *out)
        torch.cuda.synchronize()
        got = out[1].cpu().tolist()[:6 * K]
        assert got == row * 6, (K, got)
        want = np.zeros((1, 1, 6, 6), bool)
        want[..., row] = True
        _check_csr(*out, want, 6 * K)


def test_row_topk_equal_scores_keep_first_blocks(dev):
    nb = 45  # not a multiple of 32: a partial selection word and a partial inversion group
    s = torch.zeros(2, nb, nb, dtype=torch.bfloat16, device=dev)
    K = 7
    out = [torch.empty(1, 2, nb + 1, dtype=torch.int32, device=dev), torch.empty(2 * nb * K, dtype=torch.int32,
           device=dev), torch.empty(1, 2, nb + 1, dtype=torch.int32, device=dev),
           torch.empty(2 * nb * K, dtype=torch.int32, device=dev)]
    C().row_topk_into(s, K, 0, *out)
    want = np.zeros((1, 2, nb, nb), bool)
    want[..., :K] = True
    _check_csr(*out, want, nb * K)


def test_row_topk_random_large(dev):
    """NB = 700 (several 64-column chunks), heavy ties from coarse scores; bit-exact vs the stable sort."""
    nb, K = 700, 37
    g = torch.Generator().manual_seed(5)
    s = (torch.randint(-20, 20, (3, nb, nb), generator=g).float() / 8).to(torch.bfloat16)
    out = [torch.empty(1, 3, nb + 1, dtype=torch.int32, device=dev), torch.empty(3 * nb * K, dtype=torch.int32,
           device=dev), torch.empty(1, 3, nb + 1, dtype=torch.int32, device=dev),
           torch.empty(3 * nb * K, dtype=torch.int32, device=dev)]
    C().row_topk_into(s.to(dev), K, 0, *out)
    want = ref.row_topk_mask(f32(s).reshape(1, 3, nb, nb), K)
    _check_csr(*out, want, nb * K)


# --------------------------------------------------------------------------- VSA2 router
@pytest.mark.parametrize("R,row_norm", [(16, 1), (8, 0), (4, 1), (32, 0)])
def test_psp_scores(qkv, R, row_norm):
    log("psp R", R, "row_norm", row_norm)
    q, k, _ = qkv["gpu"]
    qr, kr, _, _, _ = C().pool_fwd(q, k, k, qkv["blk"], R)
    lse2 = C().router_lse(qr, kr, qkv["blk"], R)
    s = C().router_scores(qr, kr, lse2, qkv["blk"], R, row_norm)
    torch.cuda.synchronize()
    want = ref.psp_scores(f32(qr), f32(kr), CNT, R, row_norm).reshape(B * H, NB, NB)
    got = f32(s)
    assert np.abs(got - want).max() <= 1e-4 * max(1.0, np.abs(want).max()), np.abs(got - want).max()


@pytest.mark.parametrize("budget", [0, 1, 17, 37, 100, 1000])
def test_global_topk_bit_exact(qkv, budget):
    log("global topk budget", budget)
    q, k, _ = qkv["gpu"]
    qr, kr, _, _, _ = C().pool_fwd(q, k, k, qkv["blk"], 16)
    lse2 = C().router_lse(qr, kr, qkv["blk"], 16)
    s = C().router_scores(qr, kr, lse2, qkv["blk"], 16, 1)
    keff = min(budget, NB * NB)
    out = [torch.empty(B, H, NB + 1, dtype=torch.int32, device=s.device),
           torch.empty(max(B * H * keff, 1), dtype=torch.int32, device=s.device),
           torch.empty(B, H, NB + 1, dtype=torch.int32, device=s.device),
           torch.empty(max(B * H * keff, 1), dtype=torch.int32, device=s.device)]
    C().global_topk_into(s, budget, 0, *out)
    want = ref.global_topk_mask(f32(s).reshape(B, H, NB, NB), budget)
    _check_csr(*out, want, keff)
    # the operator-level router gives the same lists
    got = C().route(qr, kr, qkv["blk"], 16, budget, 1)
    n = B * H * keff
    assert torch.equal(got[0], out[0]) and torch.equal(got[2], out[2])
    assert torch.equal(got[1][:n], out[1][:n]) and torch.equal(got[3][:n], out[3][:n])


def test_global_topk_ties_and_signed_zero(dev):
    nb = 40
    g = torch.Generator().manual_seed(3)
    s = (torch.randint(-3, 4, (2, nb, nb), generator=g).float() / 4)
    s[0, 5, :] = -0.0
    budget = 333
    out = [torch.empty(1, 2, nb + 1, dtype=torch.int32, device=dev), torch.empty(2 * budget, dtype=torch.int32,
           device=dev), torch.empty(1, 2, nb + 1, dtype=torch.int32, device=dev),
           torch.empty(2 * budget, dtype=torch.int32, device=dev)]
    C().global_topk_into(s.to(dev), budget, 0, *out)
    want = ref.global_topk_mask(s.numpy().reshape(1, 2, nb, nb), budget)
    _check_csr(*out, want, budget)


def test_csr_transpose_and_mask_to_selection(dev):
    m = random_mask(11)
    sel = selection_of(m, dev)
    kp, ki = C().csr_transpose(sel.q2k_ptr, sel.q2k_idx)
    assert torch.equal(kp, sel.k2q_ptr) and torch.equal(ki, sel.k2q_idx)
    assert np.array_equal(sel.to_mask(NB).cpu().numpy(), m)
    assert np.array_equal(sel.col_mask(NB).cpu().numpy(), m)


# --------------------------------------------------------------------------- fine attention
@pytest.mark.parametrize("seed", [0, 1])
def test_fine_forward(qkv, seed):
    log("fine fwd seed", seed)
    q, k, v = qkv["gpu"]
    m = random_mask(seed)
    sel = selection_of(m, q.device)
    o, lse = C().attn_fwd(q, k, v, sel.q2k_ptr, sel.q2k_idx, qkv["blk"])
    torch.cuda.synchronize()
    wo, wl = ref.fine_attention(*(f32(x) for x in qkv["cpu"]), CNT, m)
    check_close("O", f32(o), wo)
    fin = np.isfinite(wl)
    assert np.array_equal(np.isfinite(f32(lse)), fin), "lse -inf pattern differs"
    check_close("lse", f32(lse)[fin], wl[fin])
    pad = ~ref.token_valid(CNT, L)
    assert (f32(o)[:, :, pad] == 0).all() and (f32(o)[:, :, 64:128] == 0).all()


def test_fine_forward_large_logits(dev):
    """Logits far from 0 and rows whose maximum rises late in the list (the deferred-rescale path)."""
    cnt = [64] * 6
    q, qd = tokens(7, dev, (1, 1, 384, 128), cnt, scale=4.0)
    k, kd = tokens(8, dev, (1, 1, 384, 128), cnt, scale=4.0)
    v, vd = tokens(9, dev, (1, 1, 384, 128), cnt)
    m = np.ones((1, 1, 6, 6), bool)
    blk = torch.tensor(cnt, dtype=torch.int32, device=dev)
    sel = selection_of(m, dev)
    o, lse = C().attn_fwd(qd, kd, vd, sel.q2k_ptr, sel.q2k_idx, blk)
    wo, wl = ref.fine_attention(f32(q), f32(k), f32(v), cnt, m)
    check_close("O", f32(o), wo)
    # logits reach |100| here; the LSE is a float32 value of that size, within the flat 2e-2
    log("large-logit lse max-abs / rel-L2", *check_close("lse", f32(lse), wl, rel=1e-3))


@pytest.mark.parametrize("seed", [0, 1])
def test_fine_backward(qkv, seed):
    log("fine bwd seed", seed)
    q, k, v = qkv["gpu"]
    m = random_mask(seed)
    sel = selection_of(m, q.device)
    o, lse = C().attn_fwd(q, k, v, sel.q2k_ptr, sel.q2k_idx, qkv["blk"])
    dout_c, dout = tokens(20 + seed, q.device)
    _, delta, _, _, _ = C().fuse_bwd(dout, o, torch.zeros(B, H, 64, D, dtype=q.dtype, device=q.device), None,
                                     qkv["blk"], 0, False)
    dk, dv = C().attn_bwd(q, k, v, dout, lse, delta, sel.k2q_ptr, sel.k2q_idx, qkv["blk"])
    dq = C().attn_bwd_q(q, k, v, dout, lse, delta, sel.q2k_ptr, sel.q2k_idx, qkv["blk"])
    torch.cuda.synchronize()
    wq, wk, wv = ref.fine_backward(*(f32(x) for x in qkv["cpu"]), CNT, m, f32(dout_c))
    check_close("dQ", f32(dq), wq)
    check_close("dK", f32(dk), wk)
    check_close("dV", f32(dv), wv)
    # the fp32 accumulate path (dq_acc += dQ) through the transposed lists gives the same dQ
    acc = torch.zeros(q.shape, dtype=torch.float32, device=q.device)
    C().attn_bwd(q, k, v, dout, lse, delta, sel.k2q_ptr, sel.k2q_idx, qkv["blk"], acc)
    check_close("dQ acc", f32(acc), wq)


# --------------------------------------------------------------------------- split-KV
def zipf_selection(seed, nb, heads, lo, hi, dev):
    g = np.random.default_rng(seed)
    m = np.zeros((1, heads, nb, nb), bool)
    for h in range(heads):
        for i in range(nb):
            n = int(min(hi, max(lo, g.zipf(1.2))))
            m[0, h, i, g.choice(nb, size=min(n, nb), replace=False)] = True
    return m


@pytest.mark.parametrize("chunk,slots,policy", [(4, 64, None), (2, 1000, None), (3, 5, None),
                                                (2, 200, (6, 1.5, 0.05, 16, 20))])
def test_split_plan_bit_exact(dev, chunk, slots, policy):
    m = zipf_selection(4, NB, 3, 1, NB, dev)
    sel = selection_of(m, dev)
    kw = {} if policy is None else dict(min_len=policy[0], rel_mean=policy[1], tail_frac=policy[2],
                                        resident=policy[3], budget=policy[4])
    tasks, merges, info = C().split_plan(sel.q2k_ptr, chunk, slots, **kw)
    t_ref, m_ref, i_ref = ref.plan_reference(sel.q2k_ptr.cpu().numpy(), chunk, slots, **kw)
    assert info.cpu().tolist() == i_ref
    assert tasks[:i_ref[0]].cpu().tolist() == t_ref
    assert merges[:i_ref[1]].cpu().tolist() == m_ref


@pytest.mark.parametrize("policy", [False, True])
def test_split_fine_equals_unsplit(qkv, policy):
    log("split fine policy", policy)
    from self_trainable_or_free_attn_amd.vsa import ops
    q, k, v = (x.detach().clone().requires_grad_(True) for x in qkv["gpu"])
    m = random_mask(3, density=0.8)
    sel = selection_of(m, q.device)
    split = ops.SplitKV.auto(chunk=2, policy=ops.SplitPolicy(rel_mean=0.5, tail_frac=0.0, fwd_waves=8.0, resident_ctas=4)) if policy \
        else ops.SplitKV(chunk=3)
    dout_c, dout = tokens(31, q.device)
    o1, l1 = ops.fine_block_sparse_attention(q, k, v, qkv["blk"], sel)
    g1 = torch.autograd.grad(o1, (q, k, v), dout)
    o2, l2 = ops.fine_block_sparse_attention(q, k, v, qkv["blk"], sel, split_kv=split)
    g2 = torch.autograd.grad(o2, (q, k, v), dout)
    rep = ops.describe_split(q, sel, split)
    assert rep["fwd"]["info"]["split_rows"] > 0, rep
    check_close("O split", f32(o2), f32(o1), max_abs=1e-2, rel=5e-3)
    fin = torch.isfinite(l1)
    assert torch.equal(fin, torch.isfinite(l2))
    check_close("lse split", f32(l2[fin]), f32(l1[fin]), max_abs=1e-3, rel=1e-4)
    wo, _ = ref.fine_attention(*(f32(x) for x in qkv["cpu"]), CNT, m)
    check_close("O split vs oracle", f32(o2), wo)
    wg = ref.fine_backward(*(f32(x) for x in qkv["cpu"]), CNT, m, f32(dout_c))
    for name, a, b, w in zip(("dQ", "dK", "dV"), g2, g1, wg):
        check_close(name + " split vs unsplit", f32(a), f32(b), max_abs=1e-2, rel=5e-3)
        check_close(name + " split vs oracle", f32(a), w)


def test_split_auto_declines_to_the_direct_kernels(qkv):
    """SplitKV.auto() on a selection where the policy splits nothing runs the direct (unsplit) kernels: outputs and
    gradients are bytes-identical to the unsplit call."""
    log("split auto declines")
    from self_trainable_or_free_attn_amd.vsa import ops
    q, k, v = (x.detach().clone().requires_grad_(True) for x in qkv["gpu"])
    sel = selection_of(random_mask(5, density=0.5), q.device)
    split = ops.SplitKV.auto()
    assert all(r["info"]["split_rows"] == 0 for r in ops.describe_split(q, sel, split).values())
    dout_c, dout = tokens(32, q.device)
    o1, l1 = ops.fine_block_sparse_attention(q, k, v, qkv["blk"], sel)
    g1 = torch.autograd.grad(o1, (q, k, v), dout)
    o2, l2 = ops.fine_block_sparse_attention(q, k, v, qkv["blk"], sel, split_kv=split)
    g2 = torch.autograd.grad(o2, (q, k, v), dout)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


# --------------------------------------------------------------------------- fusion and operators
@pytest.mark.parametrize("gate_kind,act", [(None, 0), ("token", 0), ("elem", 1)])
def test_fuse_forward_backward(qkv, gate_kind, act):
    dev = qkv["blk"].device
    of_c, of = tokens(40, dev)
    g = torch.Generator().manual_seed(41)
    oc = (torch.randn(B, H, 64, D, generator=g)).to(torch.bfloat16)
    gate = None
    if gate_kind == "token":
        gate = torch.randn(B, H, L, generator=g).to(torch.bfloat16)
    elif gate_kind == "elem":
        gate = torch.randn(B, H, L, D, generator=g).to(torch.bfloat16)
    gd = gate.to(dev) if gate is not None else None
    o = C().fuse_fwd(of, oc.to(dev), gd, qkv["blk"], act)
    dout_c, dout = tokens(42, dev)
    dof, delta_f, doc, delta_c, dgate = C().fuse_bwd(dout, of, oc.to(dev), gd, qkv["blk"], act)
    torch.cuda.synchronize()
    # float64 torch reference of O = valid (O_f + act(gate) O_c[blk])
    valid = torch.as_tensor(ref.token_valid(CNT, L))[None, None, :, None].double()
    ofx = of_c.double().requires_grad_(True)
    ocx = oc.double().requires_grad_(True)
    gx = gate.double().requires_grad_(True) if gate is not None else None
    blk = torch.arange(L) // 64
    a = torch.ones(1) if gx is None else (torch.tanh(gx) if act == 0 else gx)
    if gx is not None and gx.dim() == 3:
        a = a[..., None]
    want = (ofx + a * ocx[:, :, blk]) * valid
    # the fused output is bf16 and reaches |5| with these N(0, 1) inputs: half a bf16 step there exceeds 2e-2
    wo = want.detach().numpy()
    check_close("O", f32(o), wo, max_abs=max(2e-2, 2.0 ** -8 * np.abs(wo).max()))
    leaves = [ofx, ocx] + ([gx] if gx is not None else [])
    grads = torch.autograd.grad(want, leaves, dout_c.double())
    # dO_c is a bf16 sum over a block's rows that reaches |30|: half a bf16 step at its largest magnitude
    wdoc = grads[1][:, :, :NB].numpy()
    log("dO_c max-abs / rel-L2", *check_close("dO_c", f32(doc)[:, :, :NB], wdoc, max_abs=bf16_max_abs(wdoc)))
    if gx is not None:
        # dgate is stored in bf16 and the per-token sums reach |20|: one bf16 step there is 0.125, so the absolute
        # bound scales with the magnitude (half a step), the relative-L2 bound stays 1e-2
        w = grads[2].numpy()
        check_close("dgate", f32(dgate), w, max_abs=max(2e-2, 2.0 ** -8 * np.abs(w).max()))
    want_df = (dout_c.double() * valid * of_c.double()).sum(-1)
    # delta is a float32 row sum of exact bf16 products: the flat bounds apply
    log("delta_f max-abs / rel-L2", *check_close("delta_f", f32(delta_f), want_df.numpy()))
    want_dc = (f32(doc)[:, :, :NB].astype(np.float64) * oc.double().numpy()[:, :, :NB]).sum(-1)
    log("delta_c max-abs / rel-L2", *check_close("delta_c", f32(delta_c)[:, :, :NB], want_dc))
    assert torch.equal(dof.cpu(), (dout_c * valid.to(torch.bfloat16)))


def test_finalize(qkv):
    dev = qkv["blk"].device
    g = torch.Generator().manual_seed(50)
    acc = torch.randn(B, H, L, D, generator=g)
    add = torch.randn(B, H, 64, D, generator=g)
    out = C().finalize(acc.to(dev), add.to(dev), qkv["blk"], torch.empty(B, H, L, D, dtype=torch.bfloat16, device=dev))
    cnt = torch.tensor(CNT, dtype=torch.float32)
    blk = torch.arange(L) // 64
    want = (acc + add[:, :, blk] / cnt[blk][None, None, :, None]) * torch.as_tensor(
        ref.token_valid(CNT, L))[None, None, :, None]
    check_close("finalize", f32(out), want.numpy())


def _operator_case(qkv, which):
    from self_trainable_or_free_attn_amd.vsa import ops
    q, k, v = (x.detach().clone().requires_grad_(True) for x in qkv["gpu"])
    g = torch.Generator().manual_seed(60)
    if which == "vsa2":
        gate_c = torch.randn(B, H, L, generator=g).to(torch.bfloat16)
        gate = gate_c.to(q.device).requires_grad_(True)
        o, sel = ops.vsa2_attention(q, k, v, gate, qkv["blk"], R=16, topk=3, return_selection=True)
        act = "tanh"
    else:
        gate_c = (torch.randn(B, H, L, D, generator=g) * 0.5).to(torch.bfloat16)
        gate = gate_c.to(q.device).requires_grad_(True)
        o, sel = ops.vsa_attention(q, k, v, qkv["blk"], 4, weight=gate, return_selection=True)
        act = "identity"
    dout_c, dout = tokens(61, q.device)
    grads = torch.autograd.grad(o, (q, k, v, gate), dout)
    mask = sel.to_mask(NB).cpu().numpy()
    if which == "vsa":
        assert (mask.sum(-1) == 4).all()
    else:
        assert mask.sum() == B * H * NB * 3
    _, _, qc, kc, vc = C().pool_fwd(*qkv["gpu"], qkv["blk"], 16 if which == "vsa2" else 32)
    pooled = [f32(x)[:, :, :NB] for x in (qc, kc, vc)]
    leaves = [x.double().requires_grad_(True) for x in (*qkv["cpu"], gate_c)]
    want = ref.vsa_output(*leaves[:3], leaves[3], CNT, mask, act, pooled=pooled)
    wg = torch.autograd.grad(want, leaves, dout_c.double())
    check_close(which + " O", f32(o), want.detach().numpy())
    for name, a, w in zip(("dQ", "dK", "dV", "dgate"), grads, wg):
        check_close(which + " " + name, f32(a), w.numpy())


def test_vsa2_attention_forward_backward(qkv):
    log("vsa2_attention end to end")
    _operator_case(qkv, "vsa2")


def test_vsa_attention_forward_backward(qkv):
    log("vsa_attention end to end")
    _operator_case(qkv, "vsa")


def test_balanced_launches_concurrent_and_repeated(qkv):
    """The fine forward, KV-owner backward and dQ kernels hand the last query / key blocks of each XCD queue out at
    run time through a 64-slot counter ring: calls on two streams at once and 40 calls in a row (wrapping the ring)
    give bytes-identical outputs."""
    log("balanced launches")
    q, k, v = qkv["gpu"]
    m = random_mask(5)
    sel = selection_of(m, q.device)
    dout = tokens(31, q.device)[1]

    def run():
        o, lse = C().attn_fwd(q, k, v, sel.q2k_ptr, sel.q2k_idx, qkv["blk"])
        _, delta, _, _, _ = C().fuse_bwd(dout, o, torch.zeros(B, H, 64, D, dtype=q.dtype, device=q.device), None,
                                         qkv["blk"], 0, False)
        dk, dv = C().attn_bwd(q, k, v, dout, lse, delta, sel.k2q_ptr, sel.k2q_idx, qkv["blk"])
        dq = C().attn_bwd_q(q, k, v, dout, lse, delta, sel.q2k_ptr, sel.q2k_idx, qkv["blk"])
        return o, lse, dk, dv, dq

    want = run()
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(2)]
    got = []
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for s in streams:
        with torch.cuda.stream(s):
            got.append(run())
    for s in streams:
        torch.cuda.current_stream().wait_stream(s)
    for _ in range(40):
        last = run()
    torch.cuda.synchronize()
    for res in got + [last]:
        for a, b in zip(res, want):
            assert torch.equal(a, b)
