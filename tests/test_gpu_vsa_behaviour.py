"""Operator-level behaviour of vsa2_attention that the reference's tests/test_vsa2.py pins (:316-631), restated on this
build: query blocks with no fine edge get only the gated coarse branch; a dense mask with gate 0 is dense attention;
a second backward through a freed graph raises; budget 0 runs the router to an empty selection; an oversized budget
clamps to the dense mask; one (sample, head) never leaks into another; reruns are bitwise identical (the dQ here
has no atomics); a non-default stream gives the same results; the returned O is the caller's (overwriting it leaves
the gradients alone) and mutating a saved input makes backward raise. Float checks against float64 graphs at
max-abs 2e-2 / rel-L2 1e-2."""
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


def case(dev, B, H, nb, D, cnt, seed):
    g = torch.Generator().manual_seed(seed)
    L = nb * 64
    valid = torch.as_tensor(ref.token_valid(cnt, L))[None, None, :, None]
    q, k, v = ((torch.randn(B, H, L, D, generator=g) * valid).to(torch.bfloat16) for _ in range(3))
    gate = torch.randn(B, H, L, generator=g).to(torch.bfloat16)
    blk = torch.tensor(cnt, dtype=torch.int32, device=dev)
    return [x.to(dev) for x in (q, k, v, gate)], [x for x in (q, k, v, gate)], blk


def oracle(cpu, cnt, mask, dev, blk, R=16, dout=None):
    """float64 output (and gradients for dout) of the full operator over the frozen mask, with the kernels' pooled
    block means."""
    from self_trainable_or_free_attn_amd.vsa import _C
    q, k, v, gate = cpu
    _, _, qc, kc, vc = _C.pool_fwd(q.to(dev), k.to(dev), v.to(dev), blk, R)
    nb = q.shape[2] // 64
    pooled = [f32(x)[:, :, :nb] for x in (qc, kc, vc)]
    leaves = [x.double().requires_grad_(True) for x in cpu]
    o = ref.vsa_output(*leaves, cnt, mask, "tanh", pooled=pooled)
    grads = torch.autograd.grad(o, leaves, dout.double()) if dout is not None else None
    return o.detach().numpy(), grads


def test_zero_edge_rows_coarse_only(dev):
    log("zero-edge rows")
    from self_trainable_or_free_attn_amd.vsa import ops
    cnt = [64, 64, 64, 64, 64, 23]
    gpu, cpu, blk = case(dev, 1, 2, 6, 128, cnt, 9)
    mask = np.zeros((1, 2, 6, 6), bool)
    mask[:, :, 3, 3] = True
    sel = ops.mask_to_selection(torch.as_tensor(mask, device=dev))
    leaves = [x.clone().requires_grad_(True) for x in gpu]
    o = ops.vsa2_attention(*leaves, blk, selection=sel)
    dout = torch.randn(o.shape, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    grads = torch.autograd.grad(o, leaves, dout.to(dev))
    assert all(torch.isfinite(x.float()).all() for x in grads)
    want, wg = oracle(cpu, cnt, mask, dev, blk, dout=dout)
    check_close("O", f32(o), want)
    for name, a, w in zip(("dQ", "dK", "dV", "dgate"), grads, wg):
        check_close(name, f32(a), w.numpy())


def test_dense_mask_gate_zero_is_dense_attention(dev):
    log("dense mask, gate 0")
    from self_trainable_or_free_attn_amd.vsa import ops
    nb = 5
    gpu, cpu, blk = case(dev, 1, 2, nb, 128, [64] * nb, 4)
    q, k, v, _ = gpu
    sel = ops.mask_to_selection(torch.ones(1, 2, nb, nb, dtype=torch.bool, device=dev))
    dense = torch.nn.functional.scaled_dot_product_attention(*(x.double() for x in cpu[:3]))
    o0 = ops.vsa2_attention(q, k, v, torch.zeros(1, 2, nb * 64, dtype=q.dtype, device=dev), blk, selection=sel)
    check_close("dense, gate 0", f32(o0), dense.numpy())
    o1 = ops.vsa2_attention(q, k, v, torch.full((1, 2, nb * 64), 2.0, dtype=q.dtype, device=dev), blk,
                            selection=sel)
    assert (o1.double().cpu() - dense).abs().max() > 1e-2


def test_second_backward_without_retained_graph_raises(dev):
    from self_trainable_or_free_attn_amd.vsa import ops
    gpu, _, blk = case(dev, 1, 1, 3, 128, [64] * 3, 6)
    q = gpu[0].clone().requires_grad_(True)
    o = ops.vsa2_attention(q, gpu[1], gpu[2], gpu[3], blk, topk=1)
    o.float().sum().backward()
    with pytest.raises(RuntimeError):
        o.float().sum().backward()


def test_zero_budget_through_router(dev):
    log("budget 0")
    from self_trainable_or_free_attn_amd.vsa import ops
    cnt = [64, 17, 64, 64, 40, 64, 64, 64, 1, 64, 64, 33]
    gpu, cpu, blk = case(dev, 1, 2, 12, 128, cnt, 14)
    leaves = [x.clone().requires_grad_(True) for x in gpu]
    o, sel = ops.vsa2_attention(*leaves, blk, topk=0, return_selection=True)
    assert sel.q2k_idx.numel() == 0 and sel.k2q_idx.numel() == 0
    dout = torch.randn(o.shape, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    grads = torch.autograd.grad(o, leaves, dout.to(dev))
    want, wg = oracle(cpu, cnt, np.zeros((1, 2, 12, 12), bool), dev, blk, dout=dout)
    check_close("O", f32(o), want)
    for name, a, w in zip(("dQ", "dK", "dV", "dgate"), grads, wg):
        check_close(name, f32(a), w.numpy())


def test_budget_overflow_clamps_to_dense(dev):
    from self_trainable_or_free_attn_amd.vsa import ops
    nb, cnt = 6, [64, 64, 64, 64, 64, 29]
    gpu, cpu, blk = case(dev, 1, 2, nb, 128, cnt, 17)
    q, k, v, _ = gpu
    gate = torch.zeros(1, 2, nb * 64, dtype=q.dtype, device=dev)
    o, sel = ops.vsa2_attention(q, k, v, gate, blk, topk=nb + 100, return_selection=True)
    assert sel.to_mask(nb).all()
    wo, _ = ref.fine_attention(*(f32(x) for x in cpu[:3]), cnt, np.ones((1, 2, nb, nb), bool))
    check_close("O", f32(o), wo)


def test_head_and_sample_isolation(dev):
    log("isolation")
    from self_trainable_or_free_attn_amd.vsa import ops
    nb = 20
    cnt = [64] * 19 + [45]
    gpu, _, blk = case(dev, 2, 3, nb, 128, cnt, 18)
    q, k, v, gate = gpu
    o0, s0 = ops.vsa2_attention(q, k, v, gate, blk, topk=3, return_selection=True)
    q2, k2 = q.clone(), k.clone()
    q2[1, 2] = q2[1, 2].flip(1)
    k2[1, 2] = -k2[1, 2]
    o1, s1 = ops.vsa2_attention(q2, k2, v, gate, blk, topk=3, return_selection=True)
    m0, m1 = s0.to_mask(nb), s1.to_mask(nb)
    keep = torch.ones(2, 3, dtype=torch.bool, device=dev)
    keep[1, 2] = False
    assert torch.equal(m0[keep], m1[keep]) and torch.equal(o0[keep], o1[keep])
    assert not torch.equal(o0[1, 2], o1[1, 2])


def _run(gpu, blk, dout, **kw):
    from self_trainable_or_free_attn_amd.vsa import ops
    leaves = [x.clone().requires_grad_(True) for x in gpu]
    o, sel = ops.vsa2_attention(*leaves, blk, topk=3, return_selection=True, **kw)
    return o.detach(), sel.to_mask(blk.numel()), torch.autograd.grad(o, leaves, dout)


def test_deterministic_rerun(dev):
    log("rerun")
    nb = 18
    cnt = [64, 64, 5, 64, 64, 64, 64, 64, 37, 64, 64, 64, 64, 64, 64, 64, 12, 64]
    gpu, _, blk = case(dev, 1, 2, nb, 128, cnt, 19)
    dout = torch.randn(gpu[0].shape, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(dev)
    a, b = _run(gpu, blk, dout), _run(gpu, blk, dout)
    assert torch.equal(a[1], b[1]) and torch.equal(a[0], b[0])
    for x, y in zip(a[2], b[2]):
        assert torch.equal(x, y)


def test_non_default_stream(dev):
    log("side stream")
    nb = 12
    cnt = [64] * 11 + [50]
    gpu, _, blk = case(dev, 1, 2, nb, 128, cnt, 20)
    dout = torch.randn(gpu[0].shape, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(dev)
    want = _run(gpu, blk, dout)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        got = _run(gpu, blk, dout)
    s.synchronize()
    assert torch.equal(got[1], want[1]) and torch.equal(got[0], want[0])
    for x, y in zip(got[2], want[2]):
        assert torch.equal(x, y)


def test_output_ownership_and_input_versioning(dev):
    from self_trainable_or_free_attn_amd.vsa import ops
    nb = 10
    cnt = [64] * 9 + [31]
    gpu, _, blk = case(dev, 1, 2, nb, 128, cnt, 23)
    dout = torch.randn(gpu[0].shape, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(dev)
    sel = ops.mask_to_selection(torch.as_tensor(np.random.default_rng(6).random((1, 2, nb, nb)) < 0.4, device=dev))
    leaves = [x.clone().requires_grad_(True) for x in gpu]
    g0 = torch.autograd.grad(ops.vsa2_attention(*leaves, blk, selection=sel), leaves, dout)
    o = ops.vsa2_attention(*leaves, blk, selection=sel)
    o.detach().fill_(123.0)
    g1 = torch.autograd.grad(o, leaves, dout)
    for a, b in zip(g0, g1):
        assert torch.equal(a, b)
    leaves = [x.clone().requires_grad_(True) for x in gpu]
    o = ops.vsa2_attention(*leaves, blk, selection=sel)
    with torch.no_grad():
        leaves[1].add_(1.0)
    with pytest.raises(RuntimeError):
        torch.autograd.grad(o, leaves, dout)
