"""VSA fine attention at the full C2 shape (B = 1, H = 24, N = 30 720 = 480 blocks, D = 128, top-60 key blocks per
query block by mean-pooled score, bf16), forward and backward through the native ops, checked against a float64
restatement of the fine attention on sampled blocks: O / LSE / dQ of sampled query blocks over their selected key
blocks, dK / dV of sampled key blocks over the query blocks that selected them (each with its own full softmax
row), at max-abs 2e-2 / rel-L2 1e-2 (bf16-stored values above 4 in magnitude: half a bf16 step). The selection
itself is pinned bit for bit against the oracle's per-row top-K on the GPU's own block scores."""
import math
import sys

import numpy as np
import pytest
import torch

from helpers import bf16_max_abs, check_close, f32
from oracle import vsa_ref as ref

pytestmark = pytest.mark.gpu

B, H, N, D, TOPK = 1, 24, 30720, 128, 60
NB = N // 64
SAMPLES = [(0, 0), (239, 11), (479, 23)]  # (block, head)


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _rows(x, blocks):
    """rows of one head's [N, D] array in the listed 64-token blocks, [len(blocks) * 64, D]"""
    idx = (np.asarray(blocks)[:, None] * 64 + np.arange(64)[None, :]).reshape(-1)
    return x[idx]


def test_vsa_fine_full_c2_shape(dev):
    from self_trainable_or_free_attn_amd.vsa import _C
    log("VSA C2 full shape: inputs")
    g = torch.Generator(device=dev).manual_seed(1)
    q, k, v, dout = (torch.randn(B, H, N, D, generator=g, device=dev).to(torch.bfloat16) for _ in range(4))
    blk = torch.full((NB,), 64, dtype=torch.int32, device=dev)
    _, _, qc, kc, _ = _C.pool_fwd(q, k, v, blk, 32)
    scores = f32(_C.block_scores(qc, kc, NB))
    q2k_ptr, q2k_idx, k2q_ptr, k2q_idx = _C.route_rows(qc, kc, NB, TOPK)
    log("VSA C2 full shape: kernels")
    o, lse = _C.attn_fwd(q, k, v, q2k_ptr, q2k_idx, blk)
    delta = (dout.float() * o.float()).sum(-1).contiguous()
    dk, dv = _C.attn_bwd(q, k, v, dout, lse, delta, k2q_ptr, k2q_idx, blk)
    dq = _C.attn_bwd_q(q, k, v, dout, lse, delta, q2k_ptr, q2k_idx, blk)
    torch.cuda.synchronize()
    # selection: per-row top-K of the GPU's own scores, bit for bit
    want = ref.row_topk_mask(scores.reshape(B, H, NB, NB), TOPK)
    rp, ri = ref.csr_from_mask(want)
    assert np.array_equal(q2k_ptr.cpu().numpy(), rp) and np.array_equal(q2k_idx.cpu().numpy()[:ri.size], ri)
    qp, qi = q2k_ptr.cpu().numpy().reshape(H, NB + 1), q2k_idx.cpu().numpy()
    kp, ki = k2q_ptr.cpu().numpy().reshape(H, NB + 1), k2q_idx.cpu().numpy()
    sc = 1.0 / math.sqrt(D)
    cache = {}

    def heads(h):  # float64 [N, D] of q, k, v, dO for head h
        if h not in cache:
            cache[h] = [x[0, h].double().cpu().numpy() for x in (q, k, v, dout)]
        return cache[h]

    def row_state(i, h):
        """P, O, lse, delta of query block i (float64) over its selected key blocks"""
        Qh, Kh, Vh, DOh = heads(h)
        sel = qi[qp[h, i]:qp[h, i + 1]]
        s = Qh[i * 64:(i + 1) * 64] @ _rows(Kh, sel).T * sc
        m = s.max(1, keepdims=True)
        lz = np.log(np.exp(s - m).sum(1, keepdims=True)) + m
        p = np.exp(s - lz)
        out = p @ _rows(Vh, sel)
        dlt = (DOh[i * 64:(i + 1) * 64] * out).sum(1)
        return sel, p, out, lz[:, 0], dlt

    go, gl, gdq, gdk, gdv = (f32(x) for x in (o, lse, dq, dk, dv))
    for b, h in SAMPLES:
        log("VSA C2 full shape: oracle block", b, "head", h)
        sel, p, out, lz, dlt = row_state(b, h)
        Qh, Kh, Vh, DOh = heads(h)
        rows = slice(b * 64, (b + 1) * 64)
        check_close(f"O b{b} h{h}", go[0, h, rows], out)
        check_close(f"LSE b{b} h{h}", gl[0, h, rows], lz)
        dpv = DOh[rows] @ _rows(Vh, sel).T
        ds = p * (dpv - dlt[:, None])
        want_dq = ds @ _rows(Kh, sel) * sc
        check_close(f"dQ b{b} h{h}", gdq[0, h, rows], want_dq, max_abs=bf16_max_abs(want_dq))
        # key block b: every query block that selected it
        want_dk = np.zeros((64, D))
        want_dv = np.zeros((64, D))
        for i in ki[kp[h, b]:kp[h, b + 1]]:
            sel_i, p_i, _, _, dlt_i = row_state(int(i), h)
            c = int(np.nonzero(sel_i == b)[0][0])
            pb = p_i[:, c * 64:(c + 1) * 64]
            do_i = DOh[i * 64:(i + 1) * 64]
            dp_b = do_i @ Vh[rows].T
            ds_b = pb * (dp_b - dlt_i[:, None])
            want_dv += pb.T @ do_i
            want_dk += ds_b.T @ Qh[i * 64:(i + 1) * 64] * sc
        check_close(f"dK b{b} h{h}", gdk[0, h, rows], want_dk, max_abs=bf16_max_abs(want_dk))
        check_close(f"dV b{b} h{h}", gdv[0, h, rows], want_dv, max_abs=bf16_max_abs(want_dv))
