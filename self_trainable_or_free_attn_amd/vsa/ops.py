"""Original VSA and VSA2 operators with autograd, over the MI355X kernels (reference echosparse/vsa/ops.py).

Pipeline of one call (every stage a HIP kernel behind include/vsa_hip.h; torch only allocates and zero-fills):
  pool (router groups of R tokens, block means)  ->  coarse attention (dense over block means)
  ->  router (VSA2: PSP scores + exact global top-k; VSA: block scores + per-row top-K) ->  fine block-sparse
  attention over the selected CSR lists  ->  gate fusion O = O_fine + act(gate) * O_coarse[blk].
Backward: fusion bookkeeping (dO_f, delta, dO_c), the coarse branch backward (fp32 per-block gradients), then the
fine branch: a KV-owner pass for dK / dV and a Q-owner pass for dQ (no atomics; every variant number runs it), with
the coarse gradients spread over each block's valid tokens.

Tensor contract (the reference's): q, k, v [B, H, L, D] contiguous bf16 or fp16, L = NB * 64 in block-major order with
blk_cnt[i] (int32, 1..64) valid tokens first in block i; padding slots hold finite values, are never pooled, output 0
and get zero gradient. D is 64 or 128 (the native ops store rows with 128 columns; D = 64 is zero-padded).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _C as _native
from ._checks import nonnegative_reals, positive_ints
from .dispatch import check_bwd_variant, select_bwd_variant

GATE_ACTS = {"tanh": 0, "identity": 1}
ROW_NORMS = {"valid_groups": 0, "paper": 1}
_ROWS_POOL_R = 32  # original VSA uses only the block means of the pooling pass; R = 32 keeps its group pools small

_state = {"bwd_override": None, "tk_bwd_opts": None}


def ext():
    """The native op set (HIP library; raises on first use if it is not built)."""
    return _native


# ------------------------------------------------------------------ selections
@dataclass
class Selection:
    """Exact block selection as CSR with absolute offsets into the idx arrays."""

    q2k_ptr: torch.Tensor  # [B, H, NB + 1] int32
    q2k_idx: torch.Tensor  # [nnz] int32, kv blocks ascending per query block
    k2q_ptr: torch.Tensor  # [B, H, NB + 1] int32
    k2q_idx: torch.Tensor  # [nnz] int32, query blocks ascending per kv block

    def row_counts(self) -> torch.Tensor:
        return (self.q2k_ptr[..., 1:] - self.q2k_ptr[..., :-1]).to(torch.int64)

    def to_mask(self, nb: int) -> torch.Tensor:
        """Dense bool mask [B, H, NB, NB] of the q2k lists."""
        return _lists_to_mask(self.q2k_ptr, self.q2k_idx, nb)

    def col_mask(self, nb: int) -> torch.Tensor:
        """The mask rebuilt from the k2q lists, transposed back to [B, H, NBq, NBkv]."""
        return _lists_to_mask(self.k2q_ptr, self.k2q_idx, nb).transpose(-1, -2)


def _lists_to_mask(ptr, idx, nb):
    B, H = ptr.shape[:2]
    lens = (ptr[..., 1:] - ptr[..., :-1]).reshape(-1).to(torch.int64)
    owner = torch.repeat_interleave(torch.arange(B * H * nb, device=ptr.device), lens)
    start = int(ptr.reshape(-1)[0])
    cols = idx[start:start + owner.numel()].to(torch.int64)
    flat = torch.zeros(B * H * nb * nb, dtype=torch.bool, device=ptr.device)
    flat[owner * nb + cols] = True
    return flat.reshape(B, H, nb, nb)


def mask_to_selection(mask: torch.Tensor) -> Selection:
    """Bool block mask [B, H, NB, NB] -> Selection (testing / diagnostics)."""
    assert mask.dim() == 4 and mask.dtype == torch.bool

    def lists(m):
        B, H, N, _ = m.shape
        rows = m.reshape(-1, N)
        ends = torch.cumsum(rows.sum(1, dtype=torch.int64), 0)
        ptr = torch.cat([torch.zeros(1, dtype=torch.int64, device=m.device), ends]).to(torch.int32)
        ptr = torch.cat([ptr[:-1].reshape(B * H, N), ptr[1:].reshape(B * H, N)[:, -1:]], 1)
        return ptr.reshape(B, H, N + 1).contiguous(), rows.nonzero()[:, 1].to(torch.int32).contiguous()

    q2k_ptr, q2k_idx = lists(mask)
    k2q_ptr, k2q_idx = lists(mask.transpose(-1, -2).contiguous())
    return Selection(q2k_ptr, q2k_idx, k2q_ptr, k2q_idx)


def budget_from_topk(nb: int, topk: Optional[int], budget: Optional[int]) -> int:
    if budget is not None:
        return int(budget)
    if topk is None:
        raise ValueError("pass topk (average kv blocks per query block) or budget")
    return int(nb) * int(topk)


def route(q, k, blk_cnt, R=16, topk=None, budget=None, row_norm="paper", max_score_bytes=2 << 30) -> Selection:
    """VSA2 router alone (stop-gradient): PSP scores over R-token groups and the exact global top-k."""
    C = ext()
    nb = q.shape[2] // 64
    blk_cnt = blk_cnt.to(torch.int32).contiguous()
    qr, kr, _, _, _ = C.pool_fwd(q, k, k, blk_cnt, R)
    return Selection(*C.route(qr, kr, blk_cnt, R, budget_from_topk(nb, topk, budget), ROW_NORMS[row_norm],
                              max_score_bytes))


def route_rows(q, k, blk_cnt, topk, max_score_bytes=2 << 30) -> Selection:
    """Original-VSA router alone (stop-gradient): whole-block scores, exactly min(topk, NB) blocks per row."""
    C = ext()
    blk_cnt = blk_cnt.to(torch.int32).contiguous()
    _, _, qc, kc, _ = C.pool_fwd(q, k, k, blk_cnt, _ROWS_POOL_R)
    return Selection(*C.route_rows(qc, kc, q.shape[2] // 64, int(topk), int(max_score_bytes)))


# ------------------------------------------------------------------ backend / variant choice
def resolve_backend(backend: str, q: torch.Tensor) -> bool:
    """False: the HIP fine kernels (the only ones built). "tk" names the SM90 ThunderKittens path, absent here."""
    if backend == "tk":
        raise RuntimeError("the tk backend requires an sm_90 GPU, bf16 inputs and an ECHOSPARSE_VSA_TK=1 build")
    if backend not in ("auto", "generic"):
        raise ValueError(f"unknown backend {backend!r}")
    return False


def set_bwd_variant(v: Optional[int]) -> None:
    """Process-wide backward variant override; None restores the automatic rule."""
    _state["bwd_override"] = None if v is None else check_bwd_variant(v, "set_bwd_variant")


def resolve_bwd_variant(q: torch.Tensor, call: Optional[int] = None) -> Tuple[int, str]:
    B, H, L, D = q.shape
    return select_bwd_variant(B, H, L, D, -1, call=call, override=_state["bwd_override"])


TK_BWD_STORE_KV = 16
TK_BWD_OPTS = (0, 1, 2, 3, 16, 17, 18, 19)


def set_tk_bwd_opts(v: Optional[int]) -> None:
    """Accepted for API parity (validated); the TK backward does not exist on this build."""
    if v is not None and v not in TK_BWD_OPTS:
        raise ValueError(f"set_tk_bwd_opts must be one of {TK_BWD_OPTS}, got {v!r}")
    _state["tk_bwd_opts"] = v


# ------------------------------------------------------------------ split-KV
@dataclass(frozen=True)
class SplitPolicy:
    """GPU-side choice of the lists worth splitting, per direction (reference ops.py:248-324 semantics): a list of n
    blocks is eligible when n >= max(min_chunks * chunk, chunk + 1, rel_mean * its head's mean list length,
    tail_frac * all edges / resident workgroups); nothing is split in a direction with more than waves * resident
    eligible lists; at most max_task_waves * resident chunk tasks per plan."""

    rel_mean: float = 4.0
    tail_frac: float = 0.05
    min_chunks: int = 2
    fwd_waves: float = 1.0
    bwd_waves: float = 8.0
    max_task_waves: int = 64
    resident_ctas: Optional[int] = None

    def __post_init__(self):
        nonnegative_reals(self, "rel_mean", "tail_frac", "fwd_waves", "bwd_waves")
        positive_ints(self, "min_chunks", "max_task_waves", "resident_ctas", optional=("resident_ctas",))


@dataclass(frozen=True)
class SplitKV:
    """Balanced split-KV scheduling of the fine attention: a selected list runs as ceil(n / chunk) chunk tasks whose
    fp32 partials are merged in a fixed order (forward: LSE merge; backward: ordered sums). Manual (policy None):
    every list longer than ``chunk``; ``SplitKV.auto()``: the SplitPolicy decides on the GPU."""

    chunk: int = 64
    fwd: bool = True
    bwd: bool = True
    max_scratch_bytes: int = 1 << 30
    policy: Optional[SplitPolicy] = None

    def __post_init__(self):
        problems = [(not 1 <= int(self.chunk) <= 1 << 30, ValueError,
                     f"SplitKV.chunk must be in [1, 2**30], got {self.chunk}"),
                    (int(self.max_scratch_bytes) < 0, ValueError, "SplitKV.max_scratch_bytes must be >= 0"),
                    (not isinstance(self.policy, (SplitPolicy, type(None))), TypeError,
                     "SplitKV.policy must be a SplitPolicy or None")]
        for bad, kind, msg in problems:
            if bad:
                raise kind(msg)

    @classmethod
    def auto(cls, chunk: int = 64, fwd: bool = True, bwd: bool = True, max_scratch_bytes: int = 1 << 30,
             policy: Optional[SplitPolicy] = None) -> "SplitKV":
        """Both directions decided on the GPU from the selection by the SplitPolicy. A direction whose plan splits
        no list runs the direct kernels (their run-time XCD balancing is 3-5 % faster than the task kernels at
        equal work; one device-to-host read of the plan's split count per direction decides). The partial
        memory cap is 1 GiB here (the reference's 64 MiB was sized for 80 GB parts): a cap that leaves some hot
        lists unsplit leaves the launch as long as the unsplit one."""
        return cls(chunk=chunk, fwd=fwd, bwd=bwd, max_scratch_bytes=max_scratch_bytes, policy=policy or SplitPolicy())


def split_slots(nnz: int, chunk: int, slot_bytes: int, max_bytes: int) -> int:
    """Partial slots of a plan: what max_bytes holds, never more than a plan can use (2 * ceil(nnz / chunk))."""
    return max(0, min(int(max_bytes) // int(slot_bytes), 2 * (-(-int(nnz) // int(chunk)))))


# resident workgroups per CU of the consuming kernels (launch bounds / LDS of csrc/vsa_attn.hip)
_WG_PER_CU = {"fwd": 2, "bwd_kv": 1, "bwd_q": 2}


def split_resident(q, use_tk: bool, kind: str, policy: Optional[SplitPolicy] = None) -> int:
    if policy is not None and policy.resident_ctas is not None:
        return int(policy.resident_ctas)
    cus = torch.cuda.get_device_properties(q.device).multi_processor_count
    return cus * _WG_PER_CU[kind]


def split_plan_for(C, q, ptr, idx, split: SplitKV, use_tk: bool, kind: str, slot_bytes: Optional[int]):
    """(tasks, merges, info, slots) of one direction: fwd (q2k), bwd_kv (k2q), bwd_q (q2k). slot_bytes None: the
    direction keeps no partials, so the slot count only bounds the task grid."""
    chunks = -(-int(idx.numel()) // split.chunk)
    cap = (1 << 62) if slot_bytes is None else int(split.max_scratch_bytes) // int(slot_bytes)
    slots = max(0, min(cap, 2 * chunks))       # a plan needs at most nnz / chunk + (split rows) <= 2 * chunks
    pol = split.policy
    if pol is None:                            # manual: every list longer than one chunk
        return (*C.split_plan(ptr, split.chunk, slots), slots)
    resident = split_resident(q, use_tk, kind, pol)
    budget = int(resident * (pol.fwd_waves if kind == "fwd" else pol.bwd_waves))
    per_row = -(-(ptr.shape[-1] - 1) // split.chunk)          # chunks of the longest possible list
    slots = min(slots, budget * per_row, pol.max_task_waves * resident)
    min_len = max(split.chunk + 1, pol.min_chunks * split.chunk)
    return (*C.split_plan(ptr, split.chunk, slots, min_len, pol.rel_mean, pol.tail_frac, resident, budget), slots)


def _as_split(split) -> Optional[SplitKV]:
    if split is None:
        return None
    if isinstance(split, str) and split == "auto":
        return SplitKV.auto()
    if not isinstance(split, SplitKV):
        raise TypeError(f"split_kv must be a SplitKV, 'auto' or None, got {type(split).__name__}")
    return split


def describe_split(q, selection: Selection, split: SplitKV, backend: str = "generic", bwd_variant: int = 0) -> dict:
    """The plans an operator call would build for this selection, per direction (synchronises; diagnostics)."""
    C = ext()
    D = q.shape[-1]
    B, H = selection.q2k_ptr.shape[:2]
    nb = selection.q2k_ptr.shape[-1] - 1
    kinds = []
    if split.fwd:
        kinds.append(("fwd", selection.q2k_ptr, selection.q2k_idx, 64 * (D + 1) * 4))
    if split.bwd:
        kinds.append(("bwd_kv", selection.k2q_ptr, selection.k2q_idx, 2 * 64 * D * 4))
        kinds.append(("bwd_q", selection.q2k_ptr, selection.q2k_idx, 64 * D * 4))
    names = ["tasks", "split_rows", "split_slots", "rows", "eligible_rows", "within_budget", "global_threshold",
             "edges"]
    report = {}
    for kind, ptr, idx, sb in kinds:
        _, merges, info, slots = split_plan_for(C, q, ptr, idx, split, False, kind, sb)
        info = info.tolist()
        m = merges[: info[1]].long()
        owner = m[:, 0] // nb if m.numel() else torch.zeros(0, dtype=torch.long, device=ptr.device)
        rows = torch.bincount(owner, minlength=B * H).tolist()
        chunks = (torch.bincount(owner, weights=m[:, 2].double(), minlength=B * H).long().tolist() if m.numel()
                  else [0] * (B * H))
        report[kind] = dict(info=dict(zip(names, info)), max_slots=slots, split_rows_per_head=rows,
                            split_chunks_per_head=chunks,
                            resident=split_resident(q, False, kind, split.policy) if split.policy else None)
    return report


def _declined(split: SplitKV, info) -> bool:
    """True when an automatic (policy) plan splits no list: the caller then runs the direct kernels. Reads one int
    of the device plan (a synchronisation); manual plans never decline."""
    return split.policy is not None and int(info[1].item()) == 0


# ------------------------------------------------------------------ fine branch
def _fine_forward(C, q, k, v, sel, blk_cnt, split: Optional[SplitKV]):
    """(O_f, lse) over the q2k lists, unsplit or as a split plan + ordered LSE merge."""
    if split is None or not split.fwd:
        return C.attn_fwd(q, k, v, sel[0], sel[1], blk_cnt)
    D = q.shape[-1]
    tasks, merges, info, slots = split_plan_for(C, q, sel[0], sel[1], split, False, "fwd", 64 * (D + 1) * 4)
    if _declined(split, info):
        return C.attn_fwd(q, k, v, sel[0], sel[1], blk_cnt)
    part_o = torch.empty(slots, 64, D, device=q.device, dtype=torch.float32)
    part_lse = torch.empty(slots, 64, device=q.device, dtype=torch.float32)
    of, lse = C.attn_fwd_tasks(q, k, v, sel[1], blk_cnt, tasks, info, part_o, part_lse)
    C.split_merge_fwd(part_o, part_lse, merges, info, blk_cnt, of, lse)
    return of, lse


def _fine_backward(C, q, k, v, dout, lse, delta, sel, blk_cnt, add_q, add_k, add_v, split: Optional[SplitKV]):
    """(dq, dk, dv) of the fine branch in q's dtype, each plus its optional per-block gradient spread as add / cnt."""
    q2k_ptr, q2k_idx, k2q_ptr, k2q_idx = sel
    if split is None or not split.bwd:
        dk, dv = C.attn_bwd(q, k, v, dout, lse, delta, k2q_ptr, k2q_idx, blk_cnt, None, add_k, add_v)
        dq = C.attn_bwd_q(q, k, v, dout, lse, delta, q2k_ptr, q2k_idx, blk_cnt, add_q)
        return dq, dk, dv
    D = q.shape[-1]
    f32 = dict(device=q.device, dtype=torch.float32)
    tasks, merges, info, slots = split_plan_for(C, q, k2q_ptr, k2q_idx, split, False, "bwd_kv", 2 * 64 * D * 4)
    if _declined(split, info):
        dk, dv = C.attn_bwd(q, k, v, dout, lse, delta, k2q_ptr, k2q_idx, blk_cnt, None, add_k, add_v)
    else:
        part_k, part_v = torch.empty(slots, 64, D, **f32), torch.empty(slots, 64, D, **f32)
        dk, dv = C.attn_bwd_tasks(q, k, v, dout, lse, delta, k2q_idx, blk_cnt, tasks, info, None, add_k, add_v,
                                  part_k, part_v)
        C.split_merge_sum(part_k, merges, info, add_k, blk_cnt, dk)
        C.split_merge_sum(part_v, merges, info, add_v, blk_cnt, dv)
        del part_k, part_v
    tasks, merges, info, slots = split_plan_for(C, q, q2k_ptr, q2k_idx, split, False, "bwd_q", 64 * D * 4)
    if _declined(split, info):
        dq = C.attn_bwd_q(q, k, v, dout, lse, delta, q2k_ptr, q2k_idx, blk_cnt, add_q)
    else:
        part_q = torch.empty(slots, 64, D, **f32)
        dq = C.attn_bwd_q_tasks(q, k, v, dout, lse, delta, q2k_idx, blk_cnt, tasks, info, add_q, part_q)
        C.split_merge_sum(part_q, merges, info, add_q, blk_cnt, dq)
    return dq, dk, dv


def _coarse_lists(B, H, nb, nbc_pad, device):
    """Dense CSR over the 64-row tiles of the pooled sequence: (tile counts, ptr, idx)."""
    T = nbc_pad // 64
    cnt = (nb - 64 * torch.arange(T, device=device)).clamp(max=64).to(torch.int32)
    heads = torch.arange(B * H, device=device, dtype=torch.int64)[:, None]
    ptr = (heads * T * T + torch.arange(T + 1, device=device)[None, :] * T).to(torch.int32).reshape(B, H, T + 1)
    idx = torch.arange(T, device=device, dtype=torch.int32).repeat(B * H * T)
    return cnt.contiguous(), ptr.contiguous(), idx.contiguous()


class _VsaFunction(torch.autograd.Function):
    """Coarse + routed fine attention of either algorithm. router: ("global", budget, row_norm) or ("rows", topk);
    the backward uses the selection frozen at forward."""

    @staticmethod
    def forward(ctx, q, k, v, gate, blk_cnt, R, router, gate_act, max_score_bytes, given, bwd, split):
        C = ext()
        B, H, L, D = q.shape
        nb = L // 64
        qr, kr, qc, kc, vc = C.pool_fwd(q, k, v, blk_cnt, R)
        c_cnt, c_ptr, c_idx = _coarse_lists(B, H, nb, qc.shape[2], q.device)
        oc, lse_c = C.attn_fwd(qc, kc, vc, c_ptr, c_idx, c_cnt)
        if given is not None:
            sel = (given.q2k_ptr, given.q2k_idx, given.k2q_ptr, given.k2q_idx)
        elif router[0] == "rows":
            sel = tuple(C.route_rows(qc, kc, nb, router[1], max_score_bytes))
        else:
            sel = tuple(C.route(qr, kr, blk_cnt, R, router[1], router[2], max_score_bytes))
        del qr, kr
        of, lse_f = _fine_forward(C, q, k, v, sel, blk_cnt, split)
        o = C.fuse_fwd(of, oc, gate, blk_cnt, gate_act)
        ctx.save_for_backward(q, k, v, gate, blk_cnt)
        ctx.held = dict(qc=qc, kc=kc, vc=vc, oc=oc, lse_c=lse_c, of=of, lse_f=lse_f, sel=sel,
                        coarse=(c_cnt, c_ptr, c_idx))
        ctx.gate_act, ctx.has_gate, ctx.split = gate_act, gate is not None, split
        ctx.bwd_variant, ctx.bwd_source = bwd
        ctx.mark_non_differentiable(*sel)
        return (o, *sel)

    @staticmethod
    def backward(ctx, dout, *unused):
        C = ext()
        q, k, v, gate, blk_cnt = ctx.saved_tensors
        held = ctx.held
        if held is None:
            raise RuntimeError("VSA backward frees its intermediates after the first backward; "
                               "re-run the forward instead of backward(retain_graph=True) twice")
        ctx.held = None
        dout = dout.contiguous()
        _, delta_f, dout_c, delta_c, dgate = C.fuse_bwd(dout, held["of"], held["oc"], gate if ctx.has_gate else None,
                                                        blk_cnt, ctx.gate_act, False)
        held["of"] = None
        c_cnt, c_ptr, c_idx = held["coarse"]
        qc, kc, vc = held["qc"], held["kc"], held["vc"]
        # coarse branch: fp32 per-block gradients (dense lists, so q2k == k2q)
        dkc, dvc = C.attn_bwd(qc, kc, vc, dout_c, held["lse_c"], delta_c, c_ptr, c_idx, c_cnt, None, None, None, True)
        dqc = torch.zeros(qc.shape, device=q.device, dtype=torch.float32)
        C.attn_bwd_q_acc(qc, kc, vc, dout_c, held["lse_c"], delta_c, c_ptr, c_idx, c_cnt, dqc)
        # fine branch on the frozen selection, plus the coarse gradients spread over each block's valid tokens
        dq, dk, dv = _fine_backward(C, q, k, v, dout, held["lse_f"], delta_f, held["sel"], blk_cnt, dqc, dkc, dvc,
                                    ctx.split)
        return (dq, dk, dv, dgate if ctx.has_gate else None) + (None,) * 8


def _run(q, k, v, gate, blk_cnt, R, router, gate_act, backend, selection, max_score_bytes, return_selection,
         bwd_variant, split_kv):
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous [B,H,L,D]")
    resolve_backend(backend, q)
    blk_cnt = blk_cnt.to(torch.int32).contiguous()
    gate = gate.contiguous() if gate is not None else None
    o, *sel = _VsaFunction.apply(q, k, v, gate, blk_cnt, int(R), router, GATE_ACTS[gate_act], int(max_score_bytes),
                                 selection, resolve_bwd_variant(q, bwd_variant), _as_split(split_kv))
    return (o, Selection(*sel)) if return_selection else o


def vsa2_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gate: Optional[torch.Tensor],
                   blk_cnt: torch.Tensor, *, R: int = 16, topk: Optional[int] = None, budget: Optional[int] = None,
                   row_norm: str = "paper", gate_act: str = "tanh", backend: str = "auto",
                   selection: Optional[Selection] = None, max_score_bytes: int = 2 << 30,
                   return_selection: bool = False, bwd_variant: Optional[int] = None, split_kv=None):
    """VSA2: O = O_fine + act(gate) * repeat(O_coarse). The PSP router (R-token groups, softmax over all pooled keys,
    pooled back to 64-token blocks) and the exact global top-k with budget NB * topk per (b, h) run on every call
    unless a frozen ``selection`` is given. gate: None, [B, H, L] or [B, H, L, D] pre-activation."""
    nb = q.shape[2] // 64
    router = ("global", budget_from_topk(nb, topk, budget) if selection is None else 0, ROW_NORMS[row_norm])
    return _run(q, k, v, gate, blk_cnt, R, router, gate_act, backend, selection, max_score_bytes, return_selection,
                bwd_variant, split_kv)


def vsa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, blk_cnt: torch.Tensor, topk: int, *,
                  weight: Optional[torch.Tensor] = None, backend: str = "auto", selection: Optional[Selection] = None,
                  max_score_bytes: int = 2 << 30, return_selection: bool = False, bwd_variant: Optional[int] = None,
                  split_kv: Optional[SplitKV] = None):
    """Original VSA: O = O_fine + W * repeat(O_coarse), router S = rnd(qc kc^T / sqrt(D)) with exactly min(topk, NB)
    kv blocks per query block (score desc, ties to the smaller index). ``weight``: [B, H, L, D] direct weight (no
    activation), None = 1."""
    if weight is not None and weight.shape != q.shape:
        raise ValueError(f"weight must be [B, H, L, D] like q, got {tuple(weight.shape)}")
    return _run(q, k, v, weight, blk_cnt, _ROWS_POOL_R, ("rows", int(topk)), "identity", backend, selection,
                max_score_bytes, return_selection, bwd_variant, split_kv)


class _FineFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, blk_cnt, selection, bwd, split):
        C = ext()
        sel = (selection.q2k_ptr, selection.q2k_idx, selection.k2q_ptr, selection.k2q_idx)
        of, lse = _fine_forward(C, q, k, v, sel, blk_cnt, split)
        ctx.save_for_backward(q, k, v, blk_cnt, of, lse, *sel)
        ctx.split = split
        ctx.bwd_variant, ctx.bwd_source = bwd
        return of, lse

    @staticmethod
    def backward(ctx, dout, dlse):
        C = ext()
        q, k, v, blk_cnt, of, lse, *sel = ctx.saved_tensors
        B, H, L, D = q.shape
        zeros_c = torch.zeros(B, H, (L // 64 + 63) // 64 * 64, D, device=q.device, dtype=q.dtype)
        dout = dout.contiguous()
        _, delta, _, _, _ = C.fuse_bwd(dout, of, zeros_c, None, blk_cnt, 0, False)
        dq, dk, dv = _fine_backward(C, q, k, v, dout, lse, delta, tuple(sel), blk_cnt, None, None, None, ctx.split)
        return dq, dk, dv, None, None, None, None


def fine_block_sparse_attention(q, k, v, blk_cnt, selection: Selection, backend: str = "auto",
                                bwd_variant: Optional[int] = None, split_kv: Optional[SplitKV] = None):
    """Fine branch alone (no coarse branch, no router): (O_f, lse); empty lists give O_f = 0, lse = -inf and padding
    query rows are zero."""
    resolve_backend(backend, q)
    return _FineFunction.apply(q, k, v, blk_cnt.to(torch.int32).contiguous(), selection,
                               resolve_bwd_variant(q, bwd_variant), _as_split(split_kv))
