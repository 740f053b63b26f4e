"""Split-KV at the full C5 shape (B = 1, H = 40, L = 75 648 = 1182 blocks, D = 128, Zipf(1.2) lists clipped to
[8, 512], seed 4 — the benchmark's workload): forward and backward with the manual policy (every list longer than
64 blocks runs as 64-block chunks + the ordered merges) equal the unsplit kernels (O at max-abs 1e-2 / rel-L2 5e-3,
LSE at 1e-3 / 1e-4, gradients at 1e-2 / 5e-3), and the forward rows of the two longest lists match a float64
restatement (max-abs 2e-2 / rel-L2 1e-2)."""
import math
import sys

import numpy as np
import pytest
import torch

from helpers import check_close, f32

pytestmark = pytest.mark.gpu

B, H, NB, D = 1, 40, 1182, 128


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_split_kv_full_c5_shape(dev):
    from self_trainable_or_free_attn_amd.vsa import ops
    log("C5 full shape: inputs and Zipf lists")
    g = torch.Generator(device=dev).manual_seed(4)
    q, k, v, dout = (torch.randn(B, H, NB * 64, D, device=dev, generator=g).to(torch.bfloat16) for _ in range(4))
    blk = torch.full((NB,), 64, dtype=torch.int32, device=dev)
    rng = np.random.default_rng(4)
    mask = np.zeros((B, H, NB, NB), bool)
    n = np.clip(rng.zipf(1.2, size=(B, H, NB)), 8, 512)
    for h in range(H):
        for i in range(NB):
            mask[0, h, i, rng.choice(NB, size=int(n[0, h, i]), replace=False)] = True
    sel = ops.mask_to_selection(torch.as_tensor(mask, device=dev))
    split = ops.SplitKV(chunk=64)
    assert ops.describe_split(q, sel, split)["fwd"]["info"]["split_rows"] > 1000
    outs = []
    for sk in (None, split):
        log("C5 full shape: split" if sk else "C5 full shape: unsplit")
        qg, kg, vg = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
        o, lse = ops.fine_block_sparse_attention(qg, kg, vg, blk, sel, split_kv=sk)
        grads = torch.autograd.grad(o, (qg, kg, vg), dout)
        torch.cuda.synchronize()
        outs.append((f32(o), f32(lse), [f32(x) for x in grads]))
    (o1, l1, g1), (o2, l2, g2) = outs
    check_close("O split vs unsplit", o2, o1, max_abs=1e-2, rel=5e-3)
    fin = np.isfinite(l1)
    assert np.array_equal(fin, np.isfinite(l2))
    check_close("LSE split vs unsplit", l2[fin], l1[fin], max_abs=1e-3, rel=1e-4)
    for name, a, b in zip(("dQ", "dK", "dV"), g2, g1):
        check_close(name + " split vs unsplit", a, b, max_abs=1e-2, rel=5e-3)
    # the forward rows of the two longest lists against float64
    sc = 1.0 / math.sqrt(D)
    for flat in np.argsort(n.reshape(-1))[-2:]:
        h, i = divmod(int(flat), NB)
        log("C5 full shape: oracle block", i, "head", h, "list", int(n[0, h, i]))
        cols = np.nonzero(mask[0, h, i])[0]
        idx = (cols[:, None] * 64 + np.arange(64)[None, :]).reshape(-1)
        qh = q[0, h, i * 64:(i + 1) * 64].double().cpu().numpy()
        kh, vh = k[0, h].double().cpu().numpy()[idx], v[0, h].double().cpu().numpy()[idx]
        s = qh @ kh.T * sc
        m = s.max(1, keepdims=True)
        lz = np.log(np.exp(s - m).sum(1, keepdims=True)) + m
        want = np.exp(s - lz) @ vh
        check_close(f"O split b{i} h{h}", o2[0, h, i * 64:(i + 1) * 64], want)
        check_close(f"LSE split b{i} h{h}", l2[0, h, i * 64:(i + 1) * 64], lz[:, 0])
