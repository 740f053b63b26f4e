"""LSE-guided block-sparse self-attention (EchoSparse) on MI355X: the schedule of the reference's
`echosparse/attention.py` (EchoSparseAttention, attention.py:133-330), driving the gfx950 kernel set.

Between two denoising steps the log-sum-exp (LSE) of every attention row barely changes. Each (CFG branch, layer)
keeps the previous step's LSE and uses it three ways: as a fixed softmax offset (no running maximum, no
rescaling); to sum the exponentials per kv block while computing the selected blocks (the block-probability map that
selects the next step's blocks); and to compensate skipped blocks inside the same softmax (block-mean key/value for
every skipped block, four clustered representatives for the most probable third of them).

Schedule of a (branch, layer): dense attention for the first `dense_steps - 1` steps, then one step with every
block through the fixed-offset kernel (exact output and the first map), then sparse steps that compute the top
`density` blocks of every 128-row query tile.

State model: the reference's compact one (H100 / RTX 5090, attention.py:72-130, 272-330), which is also the one that
suits 288 GB of HBM best: per layer only the offsets of each branch and the next step's selection as two bit masks
per tile; the map, the lists and the scales are scratch shared by all layers.
"""
import torch

from . import backends

BM = 128
BK = 64
LOG2E = 1.4426950408889634
MIN_BLOCKS = 64          # sequences shorter than 64 kv blocks (4096 tokens) run dense


def _cdiv(a, b):
    return -(-a // b)


def _next_pow2(n):
    return 1 << (n - 1).bit_length()


def dense_attention(q, k, v, return_lse=False):
    """Dense attention on [B, Lq, H, D] queries over [B, Lk, H, D] keys / values (bf16, D = 128) with the native
    kernel; Lk may differ from Lq (cross-attention, text rows). With return_lse also the natural-log LSE [B, H, Lq]
    (the FlashAttention-4 contract the reference calls, attention.py:33-35)."""
    from .kernels import gfx950
    B, Lq = q.shape[:2]
    outs, lses = [], []
    for b in range(B):
        if k.shape[1] == Lq:
            out, lse2 = gfx950.dense_attention(q[b], k[b], v[b])
        else:
            out, lse2 = gfx950.dense_attention_kv(q[b], k[b], v[b])
        outs.append(out)
        lses.append(lse2[:Lq].t() / LOG2E)
    out = outs[0][None] if B == 1 else torch.stack(outs)
    if not return_lse:
        return out
    return out, (lses[0][None] if B == 1 else torch.stack(lses))


class _CompactState:
    """Persistent per-layer state: a log2 softmax offset per branch and, per plan slot, a pair of bit masks (exact
    blocks, skipped blocks). Without CFG a single branch overwrites the slot it has just consumed; with CFG the
    selecting branch 0 fills the second slot for the next step, so branches 1.. of the current step keep reading an
    unchanged first slot (reference attention.py:72-96)."""

    _serial = 0

    def __init__(self, L, H, device):
        nb = _cdiv(L, BK)
        self.L, self.H, self.device = L, H, device
        _CompactState._serial += 1
        self.serial = _CompactState._serial     # identifies the layer state whose lists the plan scratch holds
        self.words = max(_next_pow2(nb) // 32, 4 * _cdiv(nb, 128))
        self.plans = []
        self.offsets = {}
        self.ready = set()          # branch ids whose offset already comes from a full-block pass
        self.current = None         # (slot, step): what this step's sparse calls read
        self.pending = None         # (slot, step): written by branch 0, consumed from the next step on

    def plan(self, i):
        while len(self.plans) <= i:
            shape = (self.H, _cdiv(self.L, BM), self.words)
            self.plans.append(tuple(torch.full(shape, -1, device=self.device, dtype=torch.int32) for _ in range(2)))
        return self.plans[i]

    def offset(self, branch):
        if branch not in self.offsets:
            self.offsets[branch] = torch.full((_cdiv(self.L, BM) * BM, self.H), 1e30, device=self.device)
        return self.offsets[branch]


class _PlanScratch:
    """Selection and list tensors for one (L, H, refine width); every layer reuses them, since only one layer's
    selection is live at a time (reference attention.py:99-116)."""

    def __init__(self, L, H, device, refine_width):
        nq, nb = _cdiv(L, BM), _cdiv(L, BK)
        self.shape = (L, H, refine_width)
        self.mass = torch.empty(H, nq, nb, device=device)
        self.keep = torch.empty(H, nq, nb, device=device, dtype=torch.uint8)
        self.next_keep = torch.empty(H, nq, nb, device=device, dtype=torch.uint8)
        self.scale_exact = torch.empty(H, nq, device=device)
        self.scale_skip = torch.empty(H, nq, device=device)
        self.counts = torch.empty(nq, H, device=device, dtype=torch.int32)
        self.blocks = torch.zeros(nq, H, nb, device=device, dtype=torch.int32)
        self.refine = torch.empty(nq, H, refine_width, device=device, dtype=torch.int32)
        self.refine_counts = torch.empty(nq, H, device=device, dtype=torch.int32)
        self.means = torch.empty(nq, H, nb, device=device, dtype=torch.int32)
        self.mean_counts = torch.empty(nq, H, device=device, dtype=torch.int32)
        self.next_offset = torch.empty(nq * BM, H, device=device)      # branch 0
        self.next_offset1 = torch.empty(nq * BM, H, device=device)     # later branches
        # the block selection's own lists (the rebuilt lists above stay valid for the later branches of the step)
        self.sel_counts = torch.empty(nq, H, device=device, dtype=torch.int32)
        self.sel_blocks = torch.zeros(nq, H, nb, device=device, dtype=torch.int32)
        self.sel_refine = torch.empty(nq, H, refine_width, device=device, dtype=torch.int32)
        self.built = None          # (layer state, plan, step) the rebuilt lists belong to


class _Buffers:
    """Block means, flags, representatives and the all-blocks lists for one (L, H, D), reused by every layer
    (reference attention.py:119-130)."""

    def __init__(self, L, H, D, device, refine_iters, K):
        nq, nb = _cdiv(L, BM), _cdiv(L, BK)
        self.shape = (L, H, D)
        # block means and tile flags: branch 0's (read by its selection on the plan stream) and the later branches'
        self.k_mean = torch.empty(nb, H, D, device=device, dtype=torch.bfloat16)
        self.v_mean = torch.empty(nb, H, D, device=device, dtype=torch.bfloat16)
        self.flags = torch.empty(nq, H, device=device, dtype=torch.int32)
        self.k_mean1 = torch.empty_like(self.k_mean)
        self.v_mean1 = torch.empty_like(self.v_mean)
        self.flags1 = torch.empty_like(self.flags)
        self.all_counts = torch.full((nq, H), nb, device=device, dtype=torch.int32)
        self.all_blocks = torch.arange(nb, device=device, dtype=torch.int32).expand(nq, H, nb).contiguous()
        self.reps = K.Representatives(L, H, D, device, iters=refine_iters)


class EchoSparseAttention:
    """Self-attention for one video at a time; call `reset()` before each video.

    `__call__(q, k, v, step, branch, layer)` takes [1, L, H, 128] bf16 tensors. `branch` numbers the transformer
    forwards of a denoising step (0: conditional, 1: unconditional); later branches reuse branch 0's block selection
    of the same step and layer. `sink`: first kv block that every query tile computes exactly. `rows`: the caller
    uses only the first `rows` output rows; the query tiles past them are skipped.

    `gpu`: "auto" (from the device of q) or "mi355x"; see `backends`.
    """

    def __init__(self, density=0.10, dense_steps=10, dense_layers=(0,), refine_iters=6, threshold=60.0, gpu="auto"):
        assert dense_steps >= 2, "the first sparse step needs the LSE of a dense step and a full-block step"
        self.density = density
        self.dense_steps = dense_steps
        self.dense_layers = set(dense_layers)
        self.refine_iters = refine_iters
        self.threshold = threshold
        backends.check_name(gpu)
        self.gpu = gpu
        self.backend = None             # resolved from the device of the first call
        self._device = None
        self.K = None
        self._states = {}
        self._buffers = None
        self._plan_scratch = None
        self._plan_stream = None        # branch 0's next-step selection runs here, overlapping later work
        self.overlap_selection = True   # False: the selection runs on the caller's stream (A/B measurements)
        # True: branch 0's selection is enqueued when the next call launches its sparse attention (and starts with
        # it), so it shares the GPU with that long kernel instead of with the next branch's representative build
        self.defer_selection = True
        self._plan_done = None          # event after the last selection's kernels
        self._pending = None            # a deferred selection: (enqueue function, event it must follow)

    def reset(self):
        self._flush_selection()
        for st in self._states.values():
            st.ready.clear()
            st.current = st.pending = None

    def __call__(self, q, k, v, step, branch, layer, sink=None, rows=None):
        B, L, H, D = q.shape
        assert B == 1, "batch size 1 only"
        if q.device != self._device:
            self._join_plan()
            self.backend = backends.resolve(self.gpu, q.device)
            self.K = backends.kernels(self.backend)
            self._states.clear()
            self._buffers = self._plan_scratch = None
            self._plan_stream = None
            self._device = q.device
        if layer in self.dense_layers or _cdiv(L, BK) < MIN_BLOCKS:
            return dense_attention(q, k, v)
        return self._call_compact(q, k, v, step, branch, layer, sink, rows)

    def _flush_selection(self, start=None):
        """Enqueue a deferred selection on the plan stream, after the event its inputs were ready at and, if given,
        after `start` (recorded on the caller's stream just before a sparse-attention launch)."""
        if self._pending is None:
            return
        enqueue, ready = self._pending
        self._pending = None
        enqueue(ready, start)

    def _join_plan(self):
        """Order the current stream after the last selection issued on the plan stream (before anything that
        writes what it reads: the plan scratch, branch 0's block means, flags and offset)."""
        self._flush_selection()
        if self._plan_done is not None:
            torch.cuda.current_stream().wait_event(self._plan_done)
            self._plan_done = None

    def _scratch(self, L, H, D, device):
        if self._buffers is None or self._buffers.shape != (L, H, D):
            self._join_plan()
            self._buffers = None                           # one sequence shape at a time
            self._buffers = _Buffers(L, H, D, device, self.refine_iters, self.K)
        return self._buffers

    def _budget(self, nb):
        """Exactly computed blocks per tile, and refined blocks (four representatives each) per tile."""
        top = max(1, int(round(self.density * nb)))
        return top, max(0, int(round((nb - top) / 3)))

    def _call_compact(self, q, k, v, step, branch, layer, sink, rows):
        L, H, D = q[0].shape
        st = self._states.get(layer)
        if st is None or st.L != L:
            self._states[layer] = None
            st = self._states[layer] = _CompactState(L, H, q.device)
        offset = st.offset(branch)
        if branch == 0 and step >= self.dense_steps:
            st.current = st.pending if st.pending is not None and st.pending[1] == step else None
            st.pending = None
        full = step == self.dense_steps - 1
        sparse = step >= self.dense_steps and branch in st.ready and st.current is not None and st.current[1] == step
        K = self.K
        # Branch 0 selects the next step's blocks on a side stream after its attention (estimate, selection, plan
        # packing, the offset update): that overlaps the later branches of the step. Every call that writes what
        # the selection reads (the plan scratch, branch 0's block means, flags and offset) waits for it first; a
        # later branch's sparse step writes none of these (its own means, flags and next offset, the rebuilt lists
        # are reused read-only).
        if branch == 0 or not sparse:
            self._join_plan()
        if not (full or sparse):
            out, lse2 = K.dense_attention(q[0], k[0], v[0])
            offset.copy_(lse2)
            return out[None]
        q, k, v = q[0], k[0], v[0]
        top, refined = self._budget(_cdiv(L, BK))
        rw = -(-refined // 32) * 32
        buf = self._scratch(L, H, D, q.device)
        ps = self._plan_scratch
        if ps is None or ps.shape != (L, H, rw):
            self._join_plan()
            self._plan_scratch = None
            ps = self._plan_scratch = _PlanScratch(L, H, q.device, rw)
        k_mean, v_mean = (buf.k_mean, buf.v_mean) if branch == 0 else (buf.k_mean1, buf.v_mean1)
        flags = buf.flags if branch == 0 else buf.flags1
        nxt = ps.next_offset if branch == 0 else ps.next_offset1
        out = torch.empty_like(q)
        if full:
            ps.keep.fill_(1)
            ps.mass.zero_()
            ps.built = None
            K.block_attention(q, k, v, out, buf.all_counts, buf.all_blocks, offset, nxt, flags,
                              mass=ps.mass, threshold=self.threshold)
            K.exact_fallback(q, k, v, out, buf.all_counts, buf.all_blocks, nxt, flags)
            K.full_step_scales(offset, nxt, ps.scale_exact, ps.scale_skip, L)
            st.ready.add(branch)
        else:
            exact, skip = st.plan(st.current[0])
            key = (st.serial, st.current[0], step)
            if ps.built != key:      # the lists of this layer's plan (a later branch reuses branch 0's)
                self._join_plan()
                K.rebuild_plan(exact, skip, ps.keep, ps.counts, ps.blocks, ps.refine, ps.refine_counts, ps.means,
                               ps.mean_counts)
                ps.built = key
            buf.reps.build(q, k, v, k_mean, v_mean)
            if branch == 0:
                ps.mass.zero_()
            start = None
            if self._pending is not None:
                start = torch.cuda.Event()
                start.record()
            K.sparse_attention(q, k, v, k_mean, v_mean, ps.means, ps.mean_counts, out, ps.counts, ps.blocks,
                               offset, nxt, flags, ps.refine, ps.refine_counts, buf.reps.k, buf.reps.v,
                               buf.reps.log_counts, mass=ps.mass if branch == 0 else None, threshold=self.threshold,
                               rows=rows)
            self._flush_selection(start)
            K.exact_fallback(q, k, v, out, ps.counts, ps.blocks, nxt, flags)
            K.compensate_fallback(q, k_mean, v_mean, ps.keep, nxt, out, flags)
        if branch != 0:
            offset.copy_(nxt)
            return out[None]
        # the next step's plan, after this step's last use of the current one in a single branch
        plan = 0 if st.current is None else st.current[0] ^ (len(st.offsets) > 1)
        exact, skip = st.plan(plan)
        main = torch.cuda.current_stream()
        if self._plan_stream is None and self.overlap_selection:
            self._plan_stream = torch.cuda.Stream(device=q.device)
        side = self._plan_stream if self.overlap_selection else main

        def enqueue(ready, start):
            # (holds q until its kernels are enqueued; record_stream keeps its memory until they have run)
            for ev in (ready, start):
                if ev is not None:
                    side.wait_event(ev)
            q.record_stream(side)
            with torch.cuda.stream(side):
                if sparse:
                    K.estimate_skipped(q, k_mean, ps.keep, offset, nxt, ps.mass, ps.scale_exact, ps.scale_skip)
                K.select_blocks(ps.mass, ps.keep, ps.scale_exact, ps.scale_skip, ps.next_keep, ps.sel_counts,
                                ps.sel_blocks, flags, skip, ps.sel_refine, top, refined, L,
                                sink=1 << 30 if sink is None else sink)
                K.pack_plan(ps.next_keep, exact)
                offset.copy_(nxt)
                self._plan_done = torch.cuda.Event()
                self._plan_done.record(side)

        ready = torch.cuda.Event()
        ready.record(main)
        if self.defer_selection and self.overlap_selection:
            self._pending = (enqueue, ready)
        else:
            enqueue(ready, None)
        st.pending = (plan, step + 1)
        return out[None]
