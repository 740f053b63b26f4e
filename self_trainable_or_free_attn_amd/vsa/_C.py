"""The VSA native op set (the reference's pybind module ``echosparse.vsa._C``, csrc/vsa/vsa2_api.cpp:904-941) over the
MI355X C ABI in include/vsa_hip.h.

Every op keeps the reference's name, argument order and return values; outputs are fresh torch tensors allocated here
(the C ABI itself never allocates), workspaces are torch uint8 tensors, and every launch goes to torch's current
stream. Shape / dtype problems raise RuntimeError with the reference's wording; there is no CPU fallback.

Differences that are not visible in results: dQ is always computed without atomics (a Q-owner pass), so ``dq_word``
only selects nothing; ``attn_bwd(..., dq_acc)`` builds the q->kv lists it needs by transposing the kv->q lists on
the device; ``route_rows`` never materialises the [NB, NB] scores, so ``max_score_bytes`` only bounds the (b, h)
chunking of ``route``.
"""
import math

import torch
import torch.nn.functional as F

from .. import _lib

BLOCK = 64
HD = 128                # columns of every token row handed to the C ABI
_FWD_VARIANT = [0]


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _tokens(x, name):
    _check(isinstance(x, torch.Tensor) and x.is_cuda, f"{name} must be a CUDA tensor")
    _check(x.dim() == 4 and x.is_contiguous(), f"{name} must be contiguous [B, H, L, D]")
    _check(x.dtype in (torch.bfloat16, torch.float16), f"{name} must be bf16 or fp16")
    _check(x.shape[3] in (64, HD), f"{name}: head dim must be 64 or 128 (this build)")
    _check(x.shape[2] % BLOCK == 0, f"{name}: L must be a multiple of 64")


def _call(name, *args):
    """Call entry point `name`, or its fp16 twin when the token tensors among the arguments are fp16 (the reference
    dispatches its kernels on the tensor dtype, vsa2_api.cpp:51); token tensors of mixed dtypes are refused."""
    dts = {a.dtype for a in args if isinstance(a, torch.Tensor) and a.dtype in (torch.bfloat16, torch.float16)}
    _check(len(dts) <= 1, f"{name}: token tensors must share one dtype (bf16 or fp16), got {sorted(map(str, dts))}")
    if dts == {torch.float16} and name in _lib.F16_TWINS:
        name += "_f16"
    _lib.call(name, *args)


def _i32(x, name):
    _check(isinstance(x, torch.Tensor) and x.is_cuda and x.dtype == torch.int32 and x.is_contiguous(),
           f"{name} must be a contiguous int32 CUDA tensor")


def _f32(x, name):
    _check(isinstance(x, torch.Tensor) and x.is_cuda and x.dtype == torch.float32 and x.is_contiguous(),
           f"{name} must be a contiguous fp32 CUDA tensor")


def _wide(x):
    """x with its last dim zero-padded to 128 columns (x itself when already 128 wide, or None). The C ABI stores
    every row with 128 columns and takes the logical head dim D (64 or 128) separately: zero columns add exact zeros
    to every dot product, and every output column past D comes out zero, so narrowing back loses nothing."""
    if x is None or x.shape[-1] == HD:
        return x
    return F.pad(x, (0, HD - x.shape[-1])).contiguous()


def _narrow(x, D):
    return x if x is None or D == HD else x[..., :D].contiguous()


class _InPlace:
    """A 128-column view of an in-place argument; put() writes its first D columns back."""

    def __init__(self, x):
        self.x, self.w = x, _wide(x)

    def put(self):
        if self.x is not None and self.w is not self.x:
            self.x.copy_(self.w[..., :self.x.shape[-1]])


def _ceil64(n):
    return (n + 63) // 64 * 64


def has_tk():
    """The ThunderKittens SM90 kernels do not exist on this build."""
    return False


def device_limits():
    """(multiprocessor count, shared memory per block) of the current device, for split planning."""
    p = torch.cuda.get_device_properties(torch.cuda.current_device())
    return [p.multi_processor_count, 160 * 1024]


def set_fwd_variant(v):
    """Kept for API parity: one forward kernel serves every shape here."""
    _FWD_VARIANT[0] = int(v)


def get_fwd_variant():
    return _FWD_VARIANT[0]


# ------------------------------------------------------------------ pooling / fusion
def pool_fwd(q, k, v, blk_cnt, R):
    """(qr, kr, qc, kc, vc): router group means and whole-block means (reference vsa2_api.cpp:73-97)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _tokens(t, n)
    _i32(blk_cnt, "blk_cnt")
    _check(R in (4, 8, 16, 32), "VSA2: router pool size R must be 4, 8, 16 or 32")
    B, H, L, D = q.shape
    NB = L // BLOCK
    _check(blk_cnt.numel() == NB, "blk_cnt must have L/64 entries")
    G = BLOCK // R
    qr = torch.zeros(B, H, _ceil64(NB * G), HD, device=q.device, dtype=q.dtype)
    kr = torch.zeros_like(qr)
    qc = torch.zeros(B, H, _ceil64(NB), HD, device=q.device, dtype=q.dtype)
    kc, vc = torch.zeros_like(qc), torch.zeros_like(qc)
    _call("vsa_pool", _wide(q), _wide(k), _wide(v), blk_cnt, qr, kr, None, qc, kc, vc, B * H, L, D, int(R))
    return [_narrow(t, D) for t in (qr, kr, qc, kc, vc)]


def fuse_fwd(of, oc, gate, blk_cnt, gate_act):
    """O = O_f + act(gate) * O_c[blk] on valid rows (reference fuse.cu:3)."""
    _tokens(of, "of")
    B, H, L, D = of.shape
    mode = 0
    if gate is not None:
        _check(gate.is_contiguous() and gate.dtype == of.dtype, "gate must be contiguous in the token dtype")
        if gate.dim() == 3 and tuple(gate.shape) == (B, H, L):
            mode = 1
        elif tuple(gate.shape) == tuple(of.shape):
            mode = 2
        else:
            raise RuntimeError("gate must be [B, H, L] or [B, H, L, D]")
    o = torch.empty(B, H, L, HD, device=of.device, dtype=of.dtype)
    _call("vsa_fuse_fwd", _wide(of), _wide(oc), _wide(gate) if mode == 2 else gate, o, blk_cnt, B * H, L, D,
              oc.shape[2], mode, int(gate_act))
    return _narrow(o, D)


def fuse_bwd(dout, of, oc, gate, blk_cnt, gate_act, write_dout_f=True):
    """(dout_f, delta_f, dout_c, delta_c, dgate) (reference fuse.cu:4-8)."""
    _tokens(dout, "dout")
    B, H, L, D = dout.shape
    mode = 0 if gate is None else (1 if gate.dim() == 3 else 2)
    dout_f = torch.empty(B, H, L, HD, device=dout.device, dtype=dout.dtype) if write_dout_f else None
    delta_f = torch.empty(B, H, L, device=dout.device, dtype=torch.float32)
    dout_c = torch.zeros(B, H, oc.shape[2], HD, device=dout.device, dtype=dout.dtype)
    delta_c = torch.zeros(B, H, oc.shape[2], device=dout.device, dtype=torch.float32)
    gate_w = _wide(gate) if mode == 2 else gate
    dgate = torch.empty_like(gate_w) if gate is not None else None
    _call("vsa_fuse_bwd", _wide(dout), _wide(of), _wide(oc), gate_w, dout_f, delta_f, dout_c,
              delta_c, dgate, blk_cnt, B * H, L, D, oc.shape[2], mode, int(gate_act))
    return _narrow(dout_f, D), delta_f, _narrow(dout_c, D), delta_c, _narrow(dgate, D) if mode == 2 else dgate


def finalize(acc, add, blk_cnt, like):
    """valid ? acc + add[blk] / cnt : 0 in like's dtype (reference fuse.cu:9)."""
    B, H, L, D = like.shape
    out = torch.empty(B, H, L, HD, dtype=like.dtype, device=blk_cnt.device)
    add_nb = add.shape[2] if add is not None else 0
    _call("vsa_finalize", _wide(acc), _wide(add), add_nb, out, blk_cnt, B * H, L, D)
    return _narrow(out, D)


# ------------------------------------------------------------------ routers
def _workspace(bh_count, NB, device):
    return torch.empty(max(1, _lib.topk_workspace_bytes(bh_count, NB)), device=device, dtype=torch.uint8)


def _block_args(qc, kc, nb):
    _check(qc.dim() == 4 and qc.shape == kc.shape, "qc/kc must be [B, H, NBc_pad, D] (pool_fwd)")
    _check(qc.shape[3] in (64, HD), "qc: head dim must be 64 or 128 (this build)")
    _check(nb >= 1 and qc.shape[2] == _ceil64(nb), "qc must hold ceil(nb/64)*64 pooled rows")


def block_scores(qc, kc, nb, bh0=0, bh_count=0):
    """Whole-block scores [bh_count, nb, nb] in the token dtype (reference vsa2_api.cpp:244-260)."""
    _block_args(qc, kc, nb)
    BH = qc.shape[0] * qc.shape[1]
    if bh_count <= 0:
        bh_count = BH - bh0
    _check(bh0 >= 0 and bh_count <= 65535 and bh0 + bh_count <= BH, "bad (b,h) range")
    scores = torch.empty(bh_count, nb, nb, device=qc.device, dtype=qc.dtype)
    _call("vsa_block_scores", _wide(qc), _wide(kc), scores, int(nb), qc.shape[2], int(bh0), int(bh_count),
              qc.shape[3])
    return scores


def _csr(B, H, NB, nnz, device):
    i32 = dict(device=device, dtype=torch.int32)
    return (torch.empty(B, H, NB + 1, **i32), torch.empty(max(nnz, 0), **i32), torch.empty(B, H, NB + 1, **i32),
            torch.empty(max(nnz, 0), **i32))


def row_topk_into(scores, topk, bh0, q2k_ptr, q2k_idx, k2q_ptr, k2q_idx):
    """Per-row top-K of given scores into rows bh0.. of the CSR outputs (reference vsa2_api.cpp:262-282)."""
    _check(scores.dim() == 3 and scores.shape[1] == scores.shape[2], "scores must be [BH, NB, NB]")
    for t, n in ((q2k_ptr, "q2k_ptr"), (q2k_idx, "q2k_idx"), (k2q_ptr, "k2q_ptr"), (k2q_idx, "k2q_idx")):
        _i32(t, n)
    bhc, NB = scores.shape[0], scores.shape[1]
    _check(bhc <= 65535, "too many (b,h) per top-k chunk")
    K = max(0, min(int(topk), NB))
    ws = _workspace(bhc, NB, scores.device)
    _call("vsa_row_topk", scores.contiguous(), NB, int(bh0), bhc, K, q2k_ptr, q2k_idx, k2q_ptr, k2q_idx, ws,
              ws.numel())


def route_rows(qc, kc, nb, topk, max_score_bytes=2 << 30):
    """Original-VSA router: (q2k_ptr, q2k_idx, k2q_ptr, k2q_idx), K = min(topk, nb) per row (reference
    vsa2_api.cpp:284-315)."""
    _block_args(qc, kc, nb)
    B, H = qc.shape[:2]
    NB, BH = int(nb), B * H
    K = max(0, min(int(topk), NB))
    _check(BH * NB * K < 2 ** 31, "VSA: total selected blocks exceed int32 CSR range")
    out = _csr(B, H, NB, BH * NB * K, qc.device)
    chunk = min(BH, 65535)
    ws = _workspace(chunk, NB, qc.device)
    D, qc, kc = qc.shape[3], _wide(qc), _wide(kc)
    for bh0 in range(0, BH, chunk):
        cnt = min(chunk, BH - bh0)
        _call("vsa_route_rows", qc, kc, NB, qc.shape[2], bh0, cnt, K, D, *out, ws, ws.numel())
    return list(out)


def router_lse(qr, kr, blk_cnt, R):
    """lse2 [B, H, Lr_pad] of every pooled query row (reference vsa2_api.cpp:122-135)."""
    B, H, Lr_pad, D = qr.shape
    lse2 = torch.empty(B, H, Lr_pad, device=qr.device, dtype=torch.float32)
    _call("vsa_router_lse", _wide(qr), _wide(kr), blk_cnt, lse2, blk_cnt.numel(), int(R), B * H, D)
    return lse2


def router_scores(qr, kr, lse2, blk_cnt, R, row_norm, bh0=0, bh_count=0):
    """PSP block scores [bh_count, NB, NB] fp32 (reference vsa2_api.cpp:137-155)."""
    B, H, _, D = qr.shape
    NB = blk_cnt.numel()
    if bh_count <= 0:
        bh_count = B * H - bh0
    scores = torch.empty(bh_count, NB, NB, device=qr.device, dtype=torch.float32)
    _call("vsa_router_scores", _wide(qr), _wide(kr), lse2, blk_cnt, scores, NB, int(R), int(row_norm), int(bh0), int(bh_count), D)
    return scores


def global_topk_into(scores, budget, bh0, q2k_ptr, q2k_idx, k2q_ptr, k2q_idx):
    """Exact global top-k of fp32 scores into rows bh0.. of the CSR outputs (reference vsa2_api.cpp:157-178)."""
    _check(scores.dtype == torch.float32 and scores.dim() == 3 and scores.shape[1] == scores.shape[2],
           "scores must be fp32 [BH, NB, NB]")
    bhc, NB = scores.shape[0], scores.shape[1]
    _check(bhc <= 65535, "too many (b,h) per top-k chunk")
    ws = _workspace(bhc, NB, scores.device)
    _call("vsa_global_topk", scores.contiguous(), NB, int(bh0), bhc, int(budget), q2k_ptr, q2k_idx, k2q_ptr,
              k2q_idx, None, ws, ws.numel())


def route(qr, kr, blk_cnt, R, budget, row_norm, max_score_bytes=2 << 30):
    """VSA2 router: lse pass, then scores + exact global top-k in (b, h) chunks bounded by max_score_bytes
    (reference vsa2_api.cpp:183-219)."""
    _i32(blk_cnt, "blk_cnt")
    B, H = qr.shape[:2]
    NB, BH = blk_cnt.numel(), B * H
    nn = NB * NB
    keff = max(0, min(int(budget), nn))
    _check(BH * keff < 2 ** 31, "VSA2: total selected blocks exceed int32 CSR range")
    out = _csr(B, H, NB, BH * keff, qr.device)
    lse2 = router_lse(qr, kr, blk_cnt, R)
    D, qr, kr = qr.shape[3], _wide(qr), _wide(kr)
    chunk = int(max(1, min(BH, int(max_score_bytes) // max(nn * 4, 1), 65535)))
    ws = _workspace(chunk, NB, qr.device)
    scores = torch.empty(chunk, NB, NB, device=qr.device, dtype=torch.float32)
    for bh0 in range(0, BH, chunk):
        cnt = min(chunk, BH - bh0)
        s = scores[:cnt]
        _call("vsa_router_scores", qr, kr, lse2, blk_cnt, s, NB, int(R), int(row_norm), bh0, cnt, D)
        _call("vsa_global_topk", s, NB, bh0, cnt, int(budget), *out, None, ws, ws.numel())
    return list(out)


def csr_transpose(ptr, idx):
    """(ptr_T, idx_T): the column lists (ascending) of a CSR selection, same absolute offsets per (b, h)."""
    B, H, n1 = ptr.shape
    NB, BH = n1 - 1, B * H
    out_ptr = torch.empty_like(ptr)
    out_idx = torch.empty_like(idx)
    chunk = min(BH, 65535)
    ws = _workspace(chunk, NB, ptr.device)
    for bh0 in range(0, BH, chunk):
        cnt = min(chunk, BH - bh0)
        _call("vsa_csr_transpose", ptr, idx, NB, bh0, cnt, out_ptr, out_idx, ws, ws.numel())
    return out_ptr, out_idx


# ------------------------------------------------------------------ attention
def _attn_args(q, k, v, blk_cnt):
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _tokens(t, n)
    _i32(blk_cnt, "blk_cnt")
    _check(q.shape == k.shape and q.shape == v.shape, "q/k/v must share [B,H,L,D] (MHA self-attention)")
    _check(blk_cnt.numel() == q.shape[2] // BLOCK, "metadata shape mismatch")


def attn_fwd(q, k, v, row_ptr, col_idx, blk_cnt, use_tk=False):
    """(o, lse): fine attention over the q2k CSR (reference vsa2_api.cpp:318-348)."""
    _attn_args(q, k, v, blk_cnt)
    _i32(row_ptr, "row_ptr")
    _i32(col_idx, "col_idx")
    B, H, L, D = q.shape
    _check(row_ptr.numel() == B * H * (L // BLOCK + 1), "metadata shape mismatch")
    o = torch.empty(B, H, L, HD, device=q.device, dtype=q.dtype)
    lse = torch.empty(B, H, L, device=q.device, dtype=torch.float32)
    _call("vsa_attn_fwd", _wide(q), _wide(k), _wide(v), row_ptr, col_idx, blk_cnt, o, lse, B * H, L, D)
    return _narrow(o, D), lse


def attn_bwd(q, k, v, dout, lse, delta, row_ptr, col_idx, blk_cnt, dq_acc=None, add_dk=None, add_dv=None,
             out_fp32=False, dq_word=False):
    """(dk, dv) over the k2q CSR, + add / cnt; with dq_acc, also dq_acc += dQ (reference vsa2_api.cpp:353-416)."""
    _attn_args(q, k, v, blk_cnt)
    B, H, L, D = q.shape
    if dq_acc is not None:
        _check(dq_acc.dtype == torch.float32 and dq_acc.shape == q.shape, "dq_acc must be fp32 like q")
    f = dict(device=q.device, dtype=torch.float32) if out_fp32 else dict(device=q.device, dtype=q.dtype)
    dk, dv = torch.empty(B, H, L, HD, **f), torch.empty(B, H, L, HD, **f)
    add_nb = add_dk.shape[2] if add_dk is not None else (add_dv.shape[2] if add_dv is not None else 0)
    q, k, v, dout = _wide(q), _wide(k), _wide(v), _wide(dout)
    _call("vsa_attn_bwd_kv", q, k, v, dout, lse, delta, row_ptr, col_idx, blk_cnt, _wide(add_dk), _wide(add_dv),
              add_nb, dk, dv, 1 if out_fp32 else 0, B * H, L, D)
    if dq_acc is not None:
        q2k_ptr, q2k_idx = csr_transpose(row_ptr, col_idx)
        acc = _InPlace(dq_acc)
        _call("vsa_attn_bwd_q", q, k, v, dout, lse, delta, q2k_ptr, q2k_idx, blk_cnt, None, 0, None, acc.w,
                  B * H, L, D)
        acc.put()
    return _narrow(dk, D), _narrow(dv, D)


def attn_bwd_q(q, k, v, dout, lse, delta, row_ptr, col_idx, blk_cnt, add_dq=None):
    """dQ over the q2k CSR without atomics, + add_dq / cnt (reference vsa2_api.cpp:419-457)."""
    _attn_args(q, k, v, blk_cnt)
    B, H, L, D = q.shape
    dq = torch.empty(B, H, L, HD, device=q.device, dtype=q.dtype)
    _call("vsa_attn_bwd_q", _wide(q), _wide(k), _wide(v), _wide(dout), lse, delta, row_ptr, col_idx, blk_cnt,
              _wide(add_dq), add_dq.shape[2] if add_dq is not None else 0, dq, None, B * H, L, D)
    return _narrow(dq, D)


# ------------------------------------------------------------------ split-KV
def split_plan(ptr, chunk, max_slots, min_len=0, rel_mean=0.0, tail_frac=0.0, resident=1, budget=-1):
    """(tasks [NR + max_slots, 4], merges [max(1, min(NR, max_slots // 2)), 4], info [8]) on the device
    (reference vsa2_api.cpp:464-508)."""
    _i32(ptr, "ptr")
    _check(ptr.dim() == 3 and ptr.shape[2] >= 2, "ptr must be [B, H, NB+1]")
    _check(1 <= chunk <= (1 << 30), "split chunk must be in [1, 2^30]")
    _check(0 <= max_slots < (1 << 30), "bad max_slots")
    _check(rel_mean >= 0.0 and tail_frac >= 0.0 and resident >= 1, "bad split policy")
    B, H, n1 = ptr.shape
    NR = B * H * (n1 - 1)
    i32 = dict(device=ptr.device, dtype=torch.int32)
    tasks = torch.empty(NR + int(max_slots), 4, **i32)
    merges = torch.empty(max(1, min(NR, int(max_slots) // 2)), 4, **i32)
    info = torch.empty(8, **i32)
    _call("vsa_split_plan", ptr, B * H, n1 - 1, int(chunk), int(max_slots), int(min_len), float(rel_mean),
              float(tail_frac), int(resident), int(budget), tasks, merges, info)
    return tasks, merges, info


def attn_fwd_tasks(q, k, v, col_idx, blk_cnt, tasks, info, part_o, part_lse):
    """(o, lse) of direct tasks; split chunks fill part_o / part_lse (reference vsa2_api.cpp:524-555)."""
    _attn_args(q, k, v, blk_cnt)
    B, H, L, D = q.shape
    _check(part_lse.numel() == part_o.numel() // D, "part_lse must be [slots, 64]")
    o = torch.empty(B, H, L, HD, device=q.device, dtype=q.dtype)
    lse = torch.empty(B, H, L, device=q.device, dtype=torch.float32)
    po = _InPlace(part_o if part_o.numel() else None)
    _call("vsa_attn_fwd_tasks", _wide(q), _wide(k), _wide(v), col_idx, blk_cnt, tasks, info, tasks.shape[0], o,
              lse, po.w, part_lse if part_lse.numel() else None, B * H, L, D)
    po.put()
    return _narrow(o, D), lse


def split_merge_fwd(part_o, part_lse, merges, info, blk_cnt, o, lse, mask_rows=True):
    """Ordered LSE merge of split rows into o / lse in place (reference vsa2_api.cpp:557-583)."""
    if part_o.numel() == 0:
        return
    B, H, L, D = o.shape
    ow = _InPlace(o)
    _call("vsa_split_merge_fwd", _wide(part_o), part_lse, merges, info, merges.shape[0], blk_cnt, ow.w, lse,
              B * H, L, D, 1 if mask_rows else 0)
    ow.put()


def split_merge_sum(part, merges, info, add, blk_cnt, out):
    """Split rows of out = sum of partials + add / cnt, in place (reference vsa2_api.cpp:586-620)."""
    if part.numel() == 0:
        return
    B, H, L, D = out.shape
    f32 = out.dtype == torch.float32
    ow = _InPlace(out)
    _call("vsa_split_merge_sum", _wide(part), merges, info, merges.shape[0], _wide(add),
              add.shape[2] if add is not None else 0, blk_cnt, None if f32 else ow.w, ow.w if f32 else None,
              B * H, L, D)
    ow.put()


def attn_bwd_tasks(q, k, v, dout, lse, delta, col_idx, blk_cnt, tasks, info, dq_acc, add_dk, add_dv, part_dk,
                   part_dv, dq_word=False):
    """(dk, dv) of direct k2q tasks; split chunks fill part_dk / part_dv (reference vsa2_api.cpp:624-685).
    dq_acc (optional) needs the q->kv lists: pass the plan's list with ``csr_transpose`` results through
    attn_bwd_q instead; here it raises, like an atomic dQ that this build does not have."""
    _check(dq_acc is None, "attn_bwd_tasks: dQ comes from attn_bwd_q_tasks on this build (no atomics)")
    _attn_args(q, k, v, blk_cnt)
    B, H, L, D = q.shape
    dk = torch.empty(B, H, L, HD, device=q.device, dtype=q.dtype)
    dv = torch.empty_like(dk)
    add_nb = add_dk.shape[2] if add_dk is not None else (add_dv.shape[2] if add_dv is not None else 0)
    pk, pv = _InPlace(part_dk if part_dk.numel() else None), _InPlace(part_dv if part_dv.numel() else None)
    _call("vsa_attn_bwd_kv_tasks", _wide(q), _wide(k), _wide(v), _wide(dout), lse, delta, col_idx, blk_cnt, tasks,
              info, tasks.shape[0], _wide(add_dk), _wide(add_dv), add_nb, dk, dv, pk.w, pv.w, B * H, L, D)
    pk.put()
    pv.put()
    return _narrow(dk, D), _narrow(dv, D)


def attn_bwd_q_tasks(q, k, v, dout, lse, delta, col_idx, blk_cnt, tasks, info, add_dq, part_dq):
    """dQ of direct q2k tasks; split chunks fill part_dq (reference vsa2_api.cpp:687-730)."""
    _attn_args(q, k, v, blk_cnt)
    B, H, L, D = q.shape
    dq = torch.empty(B, H, L, HD, device=q.device, dtype=q.dtype)
    pq = _InPlace(part_dq if part_dq.numel() else None)
    _call("vsa_attn_bwd_q_tasks", _wide(q), _wide(k), _wide(v), _wide(dout), lse, delta, col_idx, blk_cnt, tasks,
              info, tasks.shape[0], _wide(add_dq), add_dq.shape[2] if add_dq is not None else 0, dq, pq.w, B * H, L, D)
    pq.put()
    return _narrow(dq, D)


def attn_bwd_q_acc(q, k, v, dout, lse, delta, row_ptr, col_idx, blk_cnt, dq_acc):
    """dq_acc += dQ over the q2k CSR (fp32, valid rows); the deterministic stand-in for an atomic dQ accumulator."""
    _attn_args(q, k, v, blk_cnt)
    _f32(dq_acc, "dq_acc")
    B, H, L, D = q.shape
    acc = _InPlace(dq_acc)
    _call("vsa_attn_bwd_q", _wide(q), _wide(k), _wide(v), _wide(dout), lse, delta, row_ptr, col_idx, blk_cnt, None,
              0, None, acc.w, B * H, L, D)
    acc.put()
    return dq_acc


# ------------------------------------------------------------------ VSA2 three-tier representatives
def rep_build(k, v, blk_cnt, mid_reps):
    """(k_mid, v_mid, lc_mid, k_tail, v_tail, lc_tail): group means of the mid_reps contiguous groups of every block
    [B, H, ceil64(NB * RM), D], block means [B, H, ceil64(NB), D], log2 counts [NB * RM] / [NB] (reference
    experiments/vsa2_representative/csrc/rep/rep_api.cpp rep_build)."""
    _tokens(k, "k")
    _tokens(v, "v")
    B, H, L, D = k.shape
    NB, RM = L // BLOCK, int(mid_reps)
    k_mid = torch.zeros(B, H, _ceil64(NB * RM), HD, device=k.device, dtype=k.dtype)
    v_mid = torch.zeros_like(k_mid)
    k_tail = torch.zeros(B, H, _ceil64(NB), HD, device=k.device, dtype=k.dtype)
    v_tail = torch.zeros_like(k_tail)
    lc_mid = torch.empty(NB * RM, device=k.device, dtype=torch.float32)
    lc_tail = torch.empty(NB, device=k.device, dtype=torch.float32)
    _call("vsa_rep_build", _wide(k), _wide(v), blk_cnt, k_mid, v_mid, lc_mid, k_tail, v_tail, lc_tail, B * H, L, D,
              RM)
    k_mid, v_mid, k_tail, v_tail = (_narrow(t, D) for t in (k_mid, v_mid, k_tail, v_tail))
    return [k_mid, v_mid, lc_mid, k_tail, v_tail, lc_tail]


def _lc_stride(lc_mid):
    """Per-head stride of a log2-count table: 0 for one [NB * RM] table, NB * RM for [B, H, NB * RM]."""
    return 0 if lc_mid.dim() == 1 else int(lc_mid.shape[-1])


def rep_build_kmeans(k, v, blk_cnt, mid_reps, iters=5, seed=0):
    """Seeded k-means tier-B tables with the block-mean tail tables: [k_mid, v_mid, lc_mid [B, H, NB * RM] (per
    head), k_tail, v_tail, lc_tail [NB]] as rep_build, plus (counts [B, H, NB * RM] int32, labels [B, H, L]
    uint8). The three-tier benchmark construction at the HunyuanVideo shape; the reference has only the contiguous
    tables."""
    tab = rep_build(k, v, blk_cnt, mid_reps)
    B, H, L, D = k.shape
    NB, RM = L // BLOCK, int(mid_reps)
    k_mid = torch.zeros(B, H, _ceil64(NB * RM), HD, device=k.device, dtype=k.dtype)
    v_mid = torch.zeros_like(k_mid)
    lc = torch.empty(B, H, NB * RM, device=k.device, dtype=torch.float32)
    counts = torch.empty(B, H, NB * RM, device=k.device, dtype=torch.int32)
    labels = torch.empty(B, H, L, device=k.device, dtype=torch.uint8)
    _call("vsa_rep_build_kmeans", _wide(k), _wide(v), blk_cnt, k_mid, v_mid, lc, counts, labels, B * H, L, D, RM,
          int(iters), int(seed) & 0xFFFFFFFF)
    tab[0], tab[1], tab[2] = _narrow(k_mid, D), _narrow(v_mid, D), lc
    return tab, counts, labels


def route_tier_rows(qr, kr, blk_cnt, R, ka, kab, row_norm, max_score_bytes=2 << 30):
    """Per-query-block tiers over VSA2's PSP router scores: the ka best kv blocks of every query block are tier A,
    the next kab - ka tier B; same outputs as route_tiers (the benchmark construction's per-query-block split)."""
    _i32(blk_cnt, "blk_cnt")
    B, H = qr.shape[:2]
    NB, BH = blk_cnt.numel(), B * H
    ka, kab = max(0, min(int(ka), NB)), max(0, min(int(kab), NB))
    _check(ka <= kab, "need ka <= kab")
    _check(BH * NB * kab < 2 ** 31, "vsa2_rep: selected blocks exceed int32 CSR range")
    W = (NB + 31) // 32
    dev = qr.device
    i32 = dict(device=dev, dtype=torch.int32)
    a_ptr, a_idx = torch.empty(B, H, NB + 1, **i32), torch.empty(max(BH * NB * ka, 1), **i32)
    ab_ptr, ab_idx = torch.empty(B, H, NB + 1, **i32), torch.empty(max(BH * NB * kab, 1), **i32)
    bits_a = torch.zeros(B, H, NB, W, **i32)
    bits_ab = torch.zeros(B, H, NB, W, **i32)
    lse2 = router_lse(qr, kr, blk_cnt, R)
    D, qr, kr = qr.shape[3], _wide(qr), _wide(kr)
    chunk = int(max(1, min(BH, int(max_score_bytes) // max(NB * NB * 4, 1), 65535)))
    scores = torch.empty(chunk, NB, NB, device=dev, dtype=torch.float32)
    for bh0 in range(0, BH, chunk):
        cnt = min(chunk, BH - bh0)
        s = scores[:cnt]
        _call("vsa_router_scores", qr, kr, lse2, blk_cnt, s, NB, int(R), int(row_norm), bh0, cnt, D)
        _call("vsa_row_tiers", s, NB, bh0, cnt, ka, kab, a_ptr, a_idx, ab_ptr, ab_idx, bits_a, bits_ab)
    k2q_ptr, k2q_idx = csr_transpose(a_ptr, a_idx)
    b_ptr = torch.zeros(B, H, NB + 1, **i32)
    b_idx = torch.empty(max(1, BH * NB * (kab - ka)), **i32)
    _call("vsa_tier_b_lists", ab_ptr, ab_idx, a_ptr, bits_a, b_ptr, b_idx, BH, NB)
    return [a_ptr, a_idx, k2q_ptr, k2q_idx, bits_a, bits_ab, b_ptr, b_idx]


def route_tiers(qr, kr, blk_cnt, R, budget_a, budget_ab, row_norm, max_score_bytes=2 << 30):
    """VSA2's router at two budgets over one score matrix: (q2k_ptr, q2k_idx, k2q_ptr, k2q_idx) of tier A, the
    bitmaps bits_a / bits_ab [B, H, NB, ceil(NB / 32)] and the tier-B lists (b_ptr, b_idx) (reference rep_api.cpp
    route_tiers)."""
    _i32(blk_cnt, "blk_cnt")
    _check(0 <= budget_a <= budget_ab, "need 0 <= budget_a <= budget_ab")
    B, H = qr.shape[:2]
    NB, BH = blk_cnt.numel(), B * H
    nn = NB * NB
    ka, kab = max(0, min(int(budget_a), nn)), max(0, min(int(budget_ab), nn))
    _check(BH * kab < 2 ** 31, "vsa2_rep: selected blocks exceed int32 CSR range")
    W = (NB + 31) // 32
    dev = qr.device
    i32 = dict(device=dev, dtype=torch.int32)
    a_out = _csr(B, H, NB, max(BH * ka, 1), dev)
    ab_out = _csr(B, H, NB, max(BH * kab, 1), dev)
    bits_a = torch.zeros(B, H, NB, W, **i32)
    bits_ab = torch.zeros(B, H, NB, W, **i32)
    lse2 = router_lse(qr, kr, blk_cnt, R)
    D, qr, kr = qr.shape[3], _wide(qr), _wide(kr)
    chunk = int(max(1, min(BH, int(max_score_bytes) // max(nn * 4, 1), 65535)))
    ws = _workspace(chunk, NB, dev)
    scores = torch.empty(chunk, NB, NB, device=dev, dtype=torch.float32)
    for bh0 in range(0, BH, chunk):
        cnt = min(chunk, BH - bh0)
        s = scores[:cnt]
        _call("vsa_router_scores", qr, kr, lse2, blk_cnt, s, NB, int(R), int(row_norm), bh0, cnt, D)
        if kab != ka:
            _call("vsa_global_topk", s, NB, bh0, cnt, kab, *ab_out, bits_ab, ws, ws.numel())
        _call("vsa_global_topk", s, NB, bh0, cnt, ka, *a_out, bits_a, ws, ws.numel())
    b_ptr = torch.zeros(B, H, NB + 1, **i32)
    b_idx = torch.empty(max(1, BH * (kab - ka)), **i32)
    if kab != ka:
        _call("vsa_tier_b_lists", ab_out[0], ab_out[1], a_out[0], bits_a, b_ptr, b_idx, BH, NB)
    else:
        bits_ab.copy_(bits_a)
    n = BH * ka
    return [a_out[0], a_out[1][:max(n, 1)], a_out[2], a_out[3][:max(n, 1)], bits_a, bits_ab, b_ptr, b_idx]


def rep_attn_fwd(q, k, v, k_mid, v_mid, lc_mid, k_tail, v_tail, lc_tail, q2k_ptr, q2k_idx, bits_a, bits_ab, blk_cnt,
                 mid_reps, phases, diag=0):
    """(o, lse) of the three-tier attention (reference rep_api.cpp rep_attn_fwd); diag is accepted and ignored."""
    _attn_args(q, k, v, blk_cnt)
    B, H, L, D = q.shape
    o = torch.empty(B, H, L, HD, device=q.device, dtype=q.dtype)
    lse = torch.empty(B, H, L, device=q.device, dtype=torch.float32)
    _call("vsa_rep_attn_fwd", _wide(q), _wide(k), _wide(v), _wide(k_mid), _wide(v_mid), lc_mid,
              _lc_stride(lc_mid), _wide(k_tail),
              _wide(v_tail), lc_tail, q2k_ptr, q2k_idx, bits_a, bits_ab, blk_cnt, o, lse, B * H, L, D, int(mid_reps),
              int(phases))
    return _narrow(o, D), lse


def rep_attn_bwd_q(q, k, v, k_mid, v_mid, lc_mid, k_tail, v_tail, lc_tail, dout, lse, delta, q2k_ptr, q2k_idx,
                   bits_a, bits_ab, blk_cnt, dk_mid, dv_mid, dk_tail, dv_tail, mid_reps, phases, add_dq=None,
                   dq_acc=None, diag=0):
    """dQ over the tiers of `phases` (+ dq_acc + add_dq / cnt), and the representative dK / dV of tiers B and C added
    into dk_mid / dv_mid / dk_tail / dv_tail (reference rep_api.cpp rep_attn_bwd_q). Deterministic: dQ in registers,
    the tables by a KV-owner pass instead of atomics."""
    _attn_args(q, k, v, blk_cnt)
    B, H, L, D = q.shape
    dq = torch.empty(B, H, L, HD, device=q.device, dtype=q.dtype)
    q, k, v, dout = _wide(q), _wide(k), _wide(v), _wide(dout)
    k_mid, v_mid, k_tail, v_tail = _wide(k_mid), _wide(v_mid), _wide(k_tail), _wide(v_tail)
    acc = _InPlace(dq_acc)
    _call("vsa_rep_attn_bwd_q", q, k, v, k_mid, v_mid, lc_mid, _lc_stride(lc_mid), k_tail, v_tail, lc_tail, dout,
              lse, delta, q2k_ptr,
              q2k_idx, bits_a, bits_ab, blk_cnt, _wide(add_dq), add_dq.shape[2] if add_dq is not None else 0, acc.w,
              dq, B * H, L, D, int(mid_reps), int(phases))
    acc.put()
    if phases & 2:
        dkm, dvm = _InPlace(dk_mid), _InPlace(dv_mid)
        _call("vsa_rep_bwd_tables", q, dout, k_mid, v_mid, lc_mid, _lc_stride(lc_mid), lse, delta, bits_a, bits_ab,
                  dkm.w, dvm.w,
                  B * H, L, D, int(mid_reps), 2)
        dkm.put()
        dvm.put()
    if phases & 4:
        dkt, dvt = _InPlace(dk_tail), _InPlace(dv_tail)
        _call("vsa_rep_bwd_tables", q, dout, k_tail, v_tail, lc_tail, 0, lse, delta, bits_a, bits_ab, dkt.w, dvt.w,
                  B * H, L, D, int(mid_reps), 4)
        dkt.put()
        dvt.put()
    return _narrow(dq, D)


def tier_a_bwd_kv(q, k, v, dout, lse, delta, k2q_ptr, k2q_idx, blk_cnt, dq_acc=None):
    """fp32 (dk, dv) of the tier-A tokens over the tier-A k2q lists (reference rep_api.cpp tier_a_bwd_kv); a given
    dq_acc receives the tier-A dQ (computed without atomics)."""
    return attn_bwd(q, k, v, dout, lse, delta, k2q_ptr, k2q_idx, blk_cnt, dq_acc, None, None, True)


def rep_unpool(dk_a, dv_a, dk_mid, dv_mid, dk_tail, dv_tail, blk_cnt, like, mid_reps, labels=None,
               mid_counts=None):
    """(dk, dv) in like's dtype: tier-A gradients + the representative gradients spread as / count (over the
    contiguous groups, or over the k-means clusters given labels and mid_counts)."""
    B, H, L, D = like.shape
    dk = torch.empty(B, H, L, HD, dtype=like.dtype, device=blk_cnt.device)
    dv = torch.empty_like(dk)
    _call("vsa_rep_unpool", *(_wide(t) for t in (dk_a, dv_a, dk_mid, dv_mid, dk_tail, dv_tail)), blk_cnt, labels,
              mid_counts, dk, dv, B * H, L, D, int(mid_reps))
    return _narrow(dk, D), _narrow(dv, D)


def row_dot(a, b, blk_cnt):
    """[B, H, L] fp32 rowsum(a * b) on valid rows, 0 on padding (reference rep_api.cpp row_dot)."""
    B, H, L, D = a.shape
    out = torch.empty(B, H, L, device=a.device, dtype=torch.float32)
    _call("vsa_row_dot", _wide(a), _wide(b), blk_cnt, out, B * H, L, D)
    return out
