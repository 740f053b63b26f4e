"""VSA2 with a three-tier representative KV budget (reference experiments/vsa2_representative/vsa2_rep/ops.py).

VSA2 attends each query block to the top-ranked kv blocks of its PSP router and drops the rest. Here the dropped
blocks stay at reduced resolution: the top ``frac_full`` of all (query block, kv block) pairs keep their 64 tokens
(tier A), the next ``frac_mid`` keep ``mid_reps`` representatives each (tier B: means of contiguous 64 / mid_reps-
token groups), and every other pair keeps the block mean (tier C). A representative of c tokens is one column of
the single softmax with + log2(c) on its logit. Tiers come from VSA2's router and exact global top-k at two budgets
over one score matrix; tiers B / C are read from the two bitmaps.

This build: forward and dQ are query-owner passes over one column stream; the representative dK / dV come from a
KV-owner pass over the representative tables (no atomics, deterministic), the tier-A token dK / dV from the fine
KV-owner kernel. Both ``bwd_variant`` values run this deterministic path.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _C as _native
from ._checks import nonnegative_reals, positive_ints
from .ops import GATE_ACTS, ROW_NORMS, _coarse_lists

PHASE_A, PHASE_B, PHASE_C = 1, 2, 4
PHASE_ALL = PHASE_A | PHASE_B | PHASE_C
MID_REPS_OK = (1, 2, 4, 8, 16)


def ext():
    return _native


TABLES = ("contiguous", "kmeans")
SPLITS = ("global", "per_row")


@dataclass(frozen=True)
class RepTiers:
    """Three-tier budget; defaults 10 % full blocks, 20 % with 4 representatives, the rest as block means.

    split="global" (the reference's): fractions of all NB * NB pairs of a (b, h), taken by two exact global top-k
    selections; ``frac_full`` alone is VSA2's budget (topk = frac_full * NB). split="per_row" (the benchmark construction):
    every query block takes round(frac_full * NB) tier-A and round(frac_mid * NB) tier-B blocks of its own row.
    tables="contiguous" (the reference's): tier-B representatives are means of the mid_reps contiguous
    64 / mid_reps-token groups; tables="kmeans": means of mid_reps clusters of the block's keys from
    ``kmeans_iters`` Lloyd rounds started at seed tokens drawn with ``seed`` (the benchmark construction: 5 rounds)."""

    frac_full: float = 0.10
    frac_mid: float = 0.20
    mid_reps: int = 4
    split: str = "global"
    tables: str = "contiguous"
    kmeans_iters: int = 5
    seed: int = 0

    def __post_init__(self):
        nonnegative_reals(self, "frac_full", "frac_mid")
        if self.frac_full + self.frac_mid > 1.0 + 1e-9:
            raise ValueError(f"frac_full + frac_mid must be <= 1, got {self.frac_full} + {self.frac_mid}")
        if self.mid_reps not in MID_REPS_OK:
            raise ValueError(f"RepTiers.mid_reps must be one of {MID_REPS_OK}, got {self.mid_reps!r}")
        if self.split not in SPLITS or self.tables not in TABLES:
            raise ValueError(f"RepTiers.split must be one of {SPLITS} and tables one of {TABLES}, got "
                             f"{self.split!r} / {self.tables!r}")
        positive_ints(self, "kmeans_iters")

    def row_budgets(self, nb: int) -> Tuple[int, int]:
        """(tier-A blocks, tier-A|B blocks) of every query block under split="per_row", clamped to NB."""
        ka = min(nb, int(round(self.frac_full * nb)))
        return ka, min(nb, max(ka, int(round((self.frac_full + self.frac_mid) * nb))))

    def budgets(self, nb: int) -> Tuple[int, int]:
        """(tier-A budget, tier-A|B budget) in pairs per (b, h), both clamped to NB * NB."""
        nn = nb * nb
        ba = min(nn, int(round(self.frac_full * nn)))
        return ba, min(nn, max(ba, int(round((self.frac_full + self.frac_mid) * nn))))

    @property
    def group_tokens(self) -> int:
        return 64 // self.mid_reps


def _unpack_bits(bits: torch.Tensor, nb: int) -> torch.Tensor:
    """[..., NB, W] int32 bitmap -> [..., NB, NB] bool (bit j % 32 of word j // 32 is column j)."""
    shifts = torch.arange(32, device=bits.device, dtype=torch.int32)
    x = (bits.unsqueeze(-1) >> shifts) & 1
    return x.reshape(*bits.shape[:-1], bits.shape[-1] * 32)[..., :nb].to(torch.bool)


def pack_bits(mask: torch.Tensor) -> torch.Tensor:
    """[B, H, NB, NB] bool -> the kernels' [B, H, NB, ceil(NB / 32)] int32 bitmap (inverse of _unpack_bits)."""
    B, H, NB, _ = mask.shape
    W = (NB + 31) // 32
    padded = torch.zeros(B, H, NB, W * 32, dtype=torch.int64, device=mask.device)
    padded[..., :NB] = mask.to(torch.int64)
    words = (padded.reshape(B, H, NB, W, 32) << torch.arange(32, device=mask.device)).sum(-1)
    return torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32).contiguous()


@dataclass
class TierSelection:
    """Frozen three-tier assignment: tier-A CSR lists, the A and A|B bitmaps, and the tier-B CSR lists."""

    q2k_ptr: torch.Tensor
    q2k_idx: torch.Tensor
    k2q_ptr: torch.Tensor
    k2q_idx: torch.Tensor
    bits_a: torch.Tensor   # [B, H, NB, ceil(NB / 32)] int32
    bits_ab: torch.Tensor
    b_ptr: Optional[torch.Tensor] = None
    b_idx: Optional[torch.Tensor] = None

    def tier_masks(self, nb: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Dense bool masks [B, H, NB, NB] of tiers A, B, C (diagnostics)."""
        a = _unpack_bits(self.bits_a, nb)
        ab = _unpack_bits(self.bits_ab, nb)
        return a, ab & ~a, ~ab

    def with_tier_b(self) -> "TierSelection":
        """Fill b_ptr / b_idx from the bitmaps when a hand-made selection lacks them."""
        if self.b_ptr is not None:
            return self
        nb = self.bits_a.shape[2]
        _, mb, _ = self.tier_masks(nb)
        B, H, N, _ = mb.shape
        rows = mb.reshape(-1, N)
        ends = torch.cumsum(rows.sum(1, dtype=torch.int64), 0)
        starts = ends - rows.sum(1, dtype=torch.int64)
        ptr = torch.cat([starts.reshape(B * H, N), ends.reshape(B * H, N)[:, -1:]], 1).reshape(B, H, N + 1)
        idx = rows.nonzero()[:, 1].to(torch.int32)
        if idx.numel() == 0:
            idx = torch.zeros(1, dtype=torch.int32, device=mb.device)
        return TierSelection(self.q2k_ptr, self.q2k_idx, self.k2q_ptr, self.k2q_idx, self.bits_a, self.bits_ab,
                             ptr.to(torch.int32).contiguous(), idx.contiguous())


def _select_tiers(C, qr, kr, blk_cnt, R, tiers: RepTiers, row_norm: int, max_score_bytes: int) -> TierSelection:
    nb = blk_cnt.numel()
    if tiers.split == "per_row":
        ka, kab = tiers.row_budgets(nb)
        return TierSelection(*C.route_tier_rows(qr, kr, blk_cnt, R, ka, kab, row_norm, max_score_bytes))
    ba, bab = tiers.budgets(nb)
    return TierSelection(*C.route_tiers(qr, kr, blk_cnt, R, ba, bab, row_norm, max_score_bytes))


def route_tiers(q, k, blk_cnt, tiers: RepTiers = RepTiers(), *, R: int = 16, row_norm: str = "paper",
                max_score_bytes: int = 2 << 30) -> TierSelection:
    """VSA2's PSP router with the tier split of ``tiers``: exact global top-k at its two budgets, or the per-row
    split (stop-gradient)."""
    C = ext()
    blk_cnt = blk_cnt.to(torch.int32).contiguous()
    qr, kr, _, _, _ = C.pool_fwd(q, k, k, blk_cnt, R)
    return _select_tiers(C, qr, kr, blk_cnt, R, tiers, ROW_NORMS[row_norm], int(max_score_bytes))


def resolve_backend(backend: str, q: torch.Tensor) -> bool:
    if backend not in ("auto", "generic", "tk"):
        raise ValueError(f"backend must be one of ('auto', 'generic', 'tk'), got {backend!r}")
    if backend == "tk":
        raise RuntimeError("backend='tk' needs an sm_90 GPU, bf16 inputs and a VSA2_REP_TK=1 build")
    return False


@dataclass(frozen=True)
class _Tables:
    """How the representative tables are built: mid_reps, "contiguous" / "kmeans", k-means rounds and seed."""
    mid_reps: int = 4
    kind: str = "contiguous"
    iters: int = 5
    seed: int = 0

    @staticmethod
    def of(tiers: RepTiers) -> "_Tables":
        return _Tables(tiers.mid_reps, tiers.tables, tiers.kmeans_iters, tiers.seed)


def build_tables(k, v, blk_cnt, spec: "_Tables"):
    """(tab, labels, counts): the six representative tables and, for k-means tables, each token's cluster and the
    cluster sizes (None for contiguous tables)."""
    C = ext()
    if spec.kind == "kmeans":
        tab, counts, labels = C.rep_build_kmeans(k, v, blk_cnt, spec.mid_reps, spec.iters, spec.seed)
        return tab, labels, counts
    return C.rep_build(k, v, blk_cnt, spec.mid_reps), None, None


def _fine_forward(C, q, k, v, blk_cnt, sel: TierSelection, spec: _Tables, phases: int):
    tab, labels, counts = build_tables(k, v, blk_cnt, spec)
    o, lse = C.rep_attn_fwd(q, k, v, *tab, sel.q2k_ptr, sel.q2k_idx, sel.bits_a, sel.bits_ab, blk_cnt,
                            spec.mid_reps, phases)
    return (tab, labels, counts), o, lse


def _fine_backward(C, q, k, v, built, dout, lse, delta, blk_cnt, sel: TierSelection, mid_reps: int, phases: int,
                   add_dq=None, add_dk=None, add_dv=None):
    """(dq, dk, dv): dQ over every walked tier in one deterministic pass, tier-A token dK / dV by the fine KV-owner
    kernel, representative dK / dV by the table KV-owner passes, then spread over their tokens. ``add_*`` are
    per-block gradients (the coarse branch) folded in like block means."""
    tab, labels, counts = built
    k_mid, v_mid, lc_mid, k_tail, v_tail, lc_tail = tab
    f32 = dict(device=q.device, dtype=torch.float32)
    dk_mid, dv_mid = torch.zeros(k_mid.shape, **f32), torch.zeros(v_mid.shape, **f32)
    dk_tail, dv_tail = torch.zeros(k_tail.shape, **f32), torch.zeros(v_tail.shape, **f32)
    dk_a = dv_a = None
    if phases & PHASE_A:
        dk_a, dv_a = C.tier_a_bwd_kv(q, k, v, dout, lse, delta, sel.k2q_ptr, sel.k2q_idx, blk_cnt)
    dq = C.rep_attn_bwd_q(q, k, v, k_mid, v_mid, lc_mid, k_tail, v_tail, lc_tail, dout, lse, delta, sel.q2k_ptr,
                          sel.q2k_idx, sel.bits_a, sel.bits_ab, blk_cnt, dk_mid, dv_mid, dk_tail, dv_tail, mid_reps,
                          phases, add_dq)
    if add_dk is not None:  # the coarse rows are the tail table's rows (ceil64(NB) each)
        dk_tail += add_dk
        dv_tail += add_dv
    dk, dv = C.rep_unpool(dk_a, dv_a, dk_mid, dv_mid, dk_tail, dv_tail, blk_cnt, k, mid_reps, labels, counts)
    return dq, dk, dv


class _RepFineFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, blk_cnt, sel, spec, phases):
        C = ext()
        tab, o, lse = _fine_forward(C, q, k, v, blk_cnt, sel, spec, phases)
        ctx.save_for_backward(q, k, v, blk_cnt, o, lse)
        ctx.tab, ctx.sel, ctx.mid_reps, ctx.phases = tab, sel, spec.mid_reps, phases
        ctx.mark_non_differentiable(lse)
        return o, lse

    @staticmethod
    def backward(ctx, dout, _dlse):
        C = ext()
        q, k, v, blk_cnt, o, lse = ctx.saved_tensors
        dout = dout.contiguous()
        delta = C.row_dot(dout, o, blk_cnt)
        dq, dk, dv = _fine_backward(C, q, k, v, ctx.tab, dout, lse, delta, blk_cnt, ctx.sel, ctx.mid_reps, ctx.phases)
        ctx.tab = ctx.sel = None
        return dq, dk, dv, None, None, None, None


def rep_fine_attention(q, k, v, blk_cnt, selection: TierSelection, *, mid_reps: int = 4, phases: int = PHASE_ALL,
                       bwd_variant: int = 1, backend: str = "generic", tables: str = "contiguous",
                       kmeans_iters: int = 5, seed: int = 0):
    """Three-tier fine attention on a frozen selection: (O_fine, lse). ``phases=PHASE_A`` is VSA2's fine attention
    on the tier-A lists; ``tables`` as RepTiers.tables."""
    if tables not in TABLES:
        raise ValueError(f"tables must be one of {TABLES}, got {tables!r}")
    if bwd_variant not in (1, 2):
        raise ValueError(f"bwd_variant must be 1 or 2, got {bwd_variant!r}")
    if mid_reps not in MID_REPS_OK:
        raise ValueError(f"mid_reps must be one of {MID_REPS_OK}, got {mid_reps!r}")
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous [B,H,L,D]")
    resolve_backend(backend, q)
    spec = _Tables(int(mid_reps), tables, int(kmeans_iters), int(seed))
    return _RepFineFunction.apply(q, k, v, blk_cnt.to(torch.int32).contiguous(), selection, spec, int(phases))


class _RepAttentionFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, gate, blk_cnt, R, tiers, gate_act, row_norm, max_score_bytes, given, phases):
        C = ext()
        B, H, L, D = q.shape
        nb = L // 64
        qr, kr, qc, kc, vc = C.pool_fwd(q, k, v, blk_cnt, R)
        c_cnt, c_ptr, c_idx = _coarse_lists(B, H, nb, qc.shape[2], q.device)
        oc, lse_c = C.attn_fwd(qc, kc, vc, c_ptr, c_idx, c_cnt)
        sel = given if given is not None else _select_tiers(C, qr, kr, blk_cnt, R, tiers, row_norm, max_score_bytes)
        del qr, kr
        tab, of, lse_f = _fine_forward(C, q, k, v, blk_cnt, sel, _Tables.of(tiers), phases)
        o = C.fuse_fwd(of, oc, gate, blk_cnt, gate_act)
        ctx.save_for_backward(q, k, v, blk_cnt, gate)
        ctx.held = dict(tab=tab, sel=sel, of=of, lse_f=lse_f, qc=qc, kc=kc, vc=vc, oc=oc, lse_c=lse_c,
                        coarse=(c_cnt, c_ptr, c_idx))
        ctx.has_gate, ctx.gate_act, ctx.mid_reps, ctx.phases = gate is not None, gate_act, tiers.mid_reps, phases
        outs = (sel.q2k_ptr, sel.q2k_idx, sel.k2q_ptr, sel.k2q_idx, sel.bits_a, sel.bits_ab)
        ctx.mark_non_differentiable(*outs)
        return (o,) + outs

    @staticmethod
    def backward(ctx, dout, *unused):
        C = ext()
        q, k, v, blk_cnt, gate = ctx.saved_tensors
        h = ctx.held
        if h is None:
            raise RuntimeError("rep_attention backward frees its intermediates after the first backward")
        ctx.held = None
        dout = dout.contiguous()
        _, delta_f, dout_c, delta_c, dgate = C.fuse_bwd(dout, h["of"], h["oc"], gate if ctx.has_gate else None,
                                                        blk_cnt, ctx.gate_act, False)
        c_cnt, c_ptr, c_idx = h["coarse"]
        dkc, dvc = C.attn_bwd(h["qc"], h["kc"], h["vc"], dout_c, h["lse_c"], delta_c, c_ptr, c_idx, c_cnt, None, None,
                              None, True)
        dqc = torch.zeros(h["qc"].shape, device=q.device, dtype=torch.float32)
        C.attn_bwd_q_acc(h["qc"], h["kc"], h["vc"], dout_c, h["lse_c"], delta_c, c_ptr, c_idx, c_cnt, dqc)
        dq, dk, dv = _fine_backward(C, q, k, v, h["tab"], dout, h["lse_f"], delta_f, blk_cnt, h["sel"], ctx.mid_reps,
                                    ctx.phases, add_dq=dqc, add_dk=dkc, add_dv=dvc)
        return (dq, dk, dv, dgate if ctx.has_gate else None) + (None,) * 8


def rep_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gate: Optional[torch.Tensor],
                  blk_cnt: torch.Tensor, *, R: int = 16, tiers: RepTiers = RepTiers(), row_norm: str = "paper",
                  gate_act: str = "tanh", selection: Optional[TierSelection] = None, max_score_bytes: int = 2 << 30,
                  return_selection: bool = False, phases: int = PHASE_ALL, bwd_variant: int = 1,
                  backend: str = "generic"):
    """VSA2 with the three-tier fine branch: O = O_fine(three tiers) + act(gate) * repeat(O_coarse)."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous [B,H,L,D]")
    if bwd_variant not in (1, 2):
        raise ValueError(f"bwd_variant must be 1 or 2, got {bwd_variant!r}")
    resolve_backend(backend, q)
    gate = gate.contiguous() if gate is not None else None
    out = _RepAttentionFunction.apply(q, k, v, gate, blk_cnt.to(torch.int32).contiguous(), int(R), tiers,
                                      GATE_ACTS[gate_act], ROW_NORMS[row_norm], int(max_score_bytes), selection,
                                      int(phases))
    if return_selection:
        sel = TierSelection(*out[1:])
        return out[0], sel
    return out[0]
