"""fp16 token tensors through the VSA / VSA2 / three-tier kernels (the _f16 twins of include/vsa_hip.h, picked by
the op layer from the tensor dtype like the reference's dtype dispatch, csrc/vsa/vsa2_api.cpp:51), against the same
CPU oracle as the bf16 tests with fp16 rounding where the kernels round: pooled means, block scores, tier tables
and selections bit for bit; outputs and gradients within max-abs 2e-2 / rel-L2 1e-2 of float64 on the same fp16
inputs. Shapes as the bf16 tests: NB = 10 with partial blocks, B = 1, H = 2, D = 128."""
import sys

import numpy as np
import pytest
import torch

from helpers import check_close, f32
from oracle import vsa_ref as ref
from oracle.bf16 import round_f16
from test_gpu_vsa import CNT, NB, L, B, H, D, _check_csr, random_mask, selection_of
from test_gpu_vsa_rep import tier_masks, selection as tier_selection

pytestmark = pytest.mark.gpu


def C():
    from self_trainable_or_free_attn_amd.vsa import _C
    return _C


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def tokens16(seed, dev, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, H, L, D, generator=g) * scale
    x = (x * torch.as_tensor(ref.token_valid(CNT, L))[None, None, :, None]).to(torch.float16)
    return x, x.to(dev)


@pytest.fixture(scope="module")
def qkv16(dev):
    out = [tokens16(s, dev) for s in (1, 2, 3)]
    return dict(cpu=[o[0] for o in out], gpu=[o[1] for o in out],
                blk=torch.tensor(CNT, dtype=torch.int32, device=dev))


@pytest.mark.parametrize("R", [8, 32])
def test_pool_f16_bit_exact(qkv16, R):
    log("fp16 pool R", R)
    q, k, v = qkv16["gpu"]
    qr, kr, qc, kc, vc = C().pool_fwd(q, k, v, qkv16["blk"], R)
    torch.cuda.synchronize()
    assert qr.dtype == torch.float16 and qc.dtype == torch.float16
    G = 64 // R
    for x, g_out, b_out in ((qkv16["cpu"][0], qr, qc), (qkv16["cpu"][1], kr, kc)):
        grp, blk = ref.pool(f32(x), CNT, R, rnd=round_f16)
        assert np.array_equal(f32(g_out)[:, :, :NB * G], grp) and np.array_equal(f32(b_out)[:, :, :NB], blk)
    _, vblk = ref.pool(f32(qkv16["cpu"][2]), CNT, R, rnd=round_f16)
    assert np.array_equal(f32(vc)[:, :, :NB], vblk)


@pytest.mark.parametrize("K", [0, 3, 10])
def test_route_rows_f16(qkv16, K):
    log("fp16 route_rows K", K)
    q, k, _ = qkv16["gpu"]
    _, _, qc, kc, _ = C().pool_fwd(q, k, k, qkv16["blk"], 32)
    scores = C().block_scores(qc, kc, NB)
    got = C().route_rows(qc, kc, NB, K)
    torch.cuda.synchronize()
    assert scores.dtype == torch.float16
    want_s = ref.block_scores(f32(qc)[:, :, :NB], f32(kc)[:, :, :NB], rnd=round_f16).reshape(B * H, NB, NB)
    gs = f32(scores)
    step = np.exp2(np.floor(np.log2(np.maximum(np.abs(want_s), 2.0 ** -24))) - 10)  # one fp16 step
    assert (np.abs(gs - want_s) <= step + 1e-30).all()
    assert (gs == want_s).mean() > 0.95
    _check_csr(*got, ref.row_topk_mask(gs.reshape(B, H, NB, NB), K), NB * K)


def test_router_f16(qkv16):
    log("fp16 PSP router + global top-k")
    q, k, _ = qkv16["gpu"]
    qr, kr, _, _, _ = C().pool_fwd(q, k, k, qkv16["blk"], 16)
    lse2 = C().router_lse(qr, kr, qkv16["blk"], 16)
    s = C().router_scores(qr, kr, lse2, qkv16["blk"], 16, 1)
    torch.cuda.synchronize()
    want = ref.psp_scores(f32(qr), f32(kr), CNT, 16, 1).reshape(B * H, NB, NB)
    assert np.abs(f32(s) - want).max() <= 1e-4 * max(1.0, np.abs(want).max())
    got = C().route(qr, kr, qkv16["blk"], 16, 37, 1)
    _check_csr(*got, ref.global_topk_mask(f32(s).reshape(B, H, NB, NB), 37), 37)


@pytest.mark.parametrize("seed", [0, 1])
def test_fine_forward_backward_f16(qkv16, seed):
    log("fp16 fine fwd/bwd seed", seed)
    q, k, v = qkv16["gpu"]
    m = random_mask(seed)
    sel = selection_of(m, q.device)
    o, lse = C().attn_fwd(q, k, v, sel.q2k_ptr, sel.q2k_idx, qkv16["blk"])
    assert o.dtype == torch.float16
    wo, wl = ref.fine_attention(*(f32(x) for x in qkv16["cpu"]), CNT, m)
    check_close("O", f32(o), wo)
    fin = np.isfinite(wl)
    assert np.array_equal(np.isfinite(f32(lse)), fin)
    check_close("lse", f32(lse)[fin], wl[fin])
    dout_c, dout = tokens16(20 + seed, q.device)
    _, delta, _, _, _ = C().fuse_bwd(dout, o, torch.zeros(B, H, 64, D, dtype=q.dtype, device=q.device), None,
                                     qkv16["blk"], 0, False)
    dk, dv = C().attn_bwd(q, k, v, dout, lse, delta, sel.k2q_ptr, sel.k2q_idx, qkv16["blk"])
    dq = C().attn_bwd_q(q, k, v, dout, lse, delta, sel.q2k_ptr, sel.q2k_idx, qkv16["blk"])
    torch.cuda.synchronize()
    assert dq.dtype == dk.dtype == dv.dtype == torch.float16
    wq, wk, wv = ref.fine_backward(*(f32(x) for x in qkv16["cpu"]), CNT, m, f32(dout_c))
    check_close("dQ", f32(dq), wq)
    check_close("dK", f32(dk), wk)
    check_close("dV", f32(dv), wv)


def test_split_f16_equals_unsplit(qkv16):
    log("fp16 split-KV")
    from self_trainable_or_free_attn_amd.vsa import ops
    q, k, v = qkv16["gpu"]
    m = np.ones((B, H, NB, NB), bool)
    sel = selection_of(m, q.device)
    dout = tokens16(70, q.device)[1]
    outs = []
    for split in (None, ops.SplitKV(chunk=3)):
        qg, kg, vg = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
        o, lse = ops.fine_block_sparse_attention(qg, kg, vg, qkv16["blk"], sel, split_kv=split)
        outs.append([f32(o), f32(lse)] + [f32(g) for g in torch.autograd.grad(o, (qg, kg, vg), dout)])
    for name, a, b in zip(("O", "lse", "dQ", "dK", "dV"), outs[1], outs[0]):
        fin = np.isfinite(b)
        check_close("split " + name, a[fin], b[fin], max_abs=1e-2, rel=5e-3)


def test_vsa2_attention_f16(qkv16):
    """The operator end to end (pool, PSP router, fine branch, coarse branch, tanh gate) in fp16: forward and the
    gradients of q, k, v and the gate against a float64 graph over the same fp16 inputs and the kernels' pooled
    means."""
    log("fp16 vsa2_attention")
    from self_trainable_or_free_attn_amd.vsa import ops
    q, k, v = (x.detach().clone().requires_grad_(True) for x in qkv16["gpu"])
    g = torch.Generator().manual_seed(60)
    gate_c = torch.randn(B, H, L, generator=g).to(torch.float16)
    gate = gate_c.to(q.device).requires_grad_(True)
    o, sel = ops.vsa2_attention(q, k, v, gate, qkv16["blk"], R=16, topk=3, return_selection=True)
    assert o.dtype == torch.float16
    dout_c, dout = tokens16(61, q.device)
    grads = torch.autograd.grad(o, (q, k, v, gate), dout)
    mask = sel.to_mask(NB).cpu().numpy()
    _, _, qc, kc, vc = C().pool_fwd(*qkv16["gpu"], qkv16["blk"], 16)
    pooled = [f32(x)[:, :, :NB] for x in (qc, kc, vc)]
    leaves = [x.double().requires_grad_(True) for x in (*qkv16["cpu"], gate_c)]
    want = ref.vsa_output(*leaves[:3], leaves[3], CNT, mask, "tanh", pooled=pooled)
    wg = torch.autograd.grad(want, leaves, dout_c.double())
    check_close("vsa2 O", f32(o), want.detach().numpy())
    for name, a, w in zip(("dQ", "dK", "dV", "dgate"), grads, wg):
        check_close("vsa2 " + name, f32(a), w.numpy())


@pytest.mark.parametrize("RM", [4, 16])
def test_rep_tables_f16_bit_exact(qkv16, RM):
    log("fp16 rep_build RM", RM)
    _, k, v = qkv16["gpu"]
    km, vm, _, kt, vt, _ = C().rep_build(k, v, qkv16["blk"], RM)
    wkm, wvm, wkt, wvt, _, _ = ref.rep_tables(f32(qkv16["cpu"][1]), f32(qkv16["cpu"][2]), CNT, RM, rnd=round_f16)
    assert np.array_equal(f32(km)[:, :, :NB * RM], wkm) and np.array_equal(f32(vm)[:, :, :NB * RM], wvm)
    assert np.array_equal(f32(kt)[:, :, :NB], wkt) and np.array_equal(f32(vt)[:, :, :NB], wvt)


def test_rep_three_tiers_f16(qkv16):
    """Three tiers (64 / 4 / 1) forward and backward in fp16 against the float64 graph with the kernels' tables."""
    log("fp16 three tiers")
    from self_trainable_or_free_attn_amd.vsa import rep
    RM = 4
    q, k, v = (t.detach().clone().requires_grad_(True) for t in qkv16["gpu"])
    a, ab = tier_masks(33)
    sel = tier_selection(a, ab, q.device)
    o, lse = rep.rep_fine_attention(q, k, v, qkv16["blk"], sel, mid_reps=RM)
    assert o.dtype == torch.float16
    dout_c, dout = tokens16(40, q.device)
    grads = torch.autograd.grad(o, (q, k, v), dout)
    torch.cuda.synchronize()
    km, vm, kt, vt, _, _ = ref.rep_tables(f32(qkv16["cpu"][1]), f32(qkv16["cpu"][2]), CNT, RM, rnd=round_f16)
    x = [t.double().requires_grad_(True) for t in qkv16["cpu"]]
    wo, wl = ref.rep_fine_torch(*x, CNT, a, ab, RM, 7, tables=(km, vm, kt, vt))
    check_close("O", f32(o), wo.detach().numpy())
    wg = torch.autograd.grad(wo, x, dout_c.double())
    for name, g, w in zip(("dQ", "dK", "dV"), grads, wg):
        check_close(name, f32(g), w.numpy())


def test_mixed_dtypes_are_refused(qkv16, dev):
    q = qkv16["gpu"][0]
    kb = qkv16["gpu"][1].to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="share one dtype"):
        C().pool_fwd(q, kb, kb, qkv16["blk"], 16)
