"""Headline benchmark: the EchoSparse sparse step on one MI355X at the Wan2.1-14B shape.

Workload (the Wan2.1-14B sparse-step configuration): per layer two CFG branch calls (B = 2), H = 40, D = 128, bf16, tokens on a
21 x 45 x 80 latent grid (L = 75 600, 1182 kv blocks of 64, 591 query tiles of 128), Morton order; Q / K a
low-frequency random Fourier field plus 0.3 N(0, 1), scaled per head so the mean row-softmax entropy is 20 % of
ln L; V ~ N(0, 1). The previous step's LSE comes from a dense pass on inputs perturbed by 1 % Gaussian noise, and a
full-block step on those inputs gives the map that selects the top 10 % blocks. A timed step is one layer of a
sparse denoising step: branch 0 (plan rebuild, representatives + block means, fixed-offset attention, fallback,
compensation, estimate, selection, plan pack) and branch 1 (the same without estimate / selection).

Printed (one JSON line, rank 0): value = TFLOP/s on executed blocks over the whole layer time; ms_per_step =
ms / layer; `roofline` for the dominant kernel (the fixed-offset sparse attention) from HIP events on its stream;
the dense comparison (torch SDPA and this build's dense kernel); `cpu_baseline` = the numpy oracle on a bounded
sample of (tile, head) pairs of the same step.
"""
import argparse
import json
import math
import os
import sys
import time

import torch

PEAK_BF16 = 2.5e15
# HBM-side bytes per es_sparse_attention launch at this workload: rocprofv3 FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0
# (scale factors from a copy of known size), profiles/echosparse_sparse_attention_wan14b_traffic.md
TRAFFIC_BYTES = 4.59e10


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--heads", type=int, default=40)
    ap.add_argument("--grid", type=str, default="21,45,80")
    ap.add_argument("--density", type=float, default=0.10)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-dense", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--c4", default="baseline", choices=["baseline", "reference"],
                    help="vsa2_rep tier construction: the benchmark's (per-query-block tiers, seeded 5-round "
                         "k-means tables) or the reference's (global budgets, contiguous group means)")
    ap.add_argument("--split-policy", default="manual", choices=["manual", "auto"],
                    help="split workload: SplitKV(chunk=64) (every list over 64 blocks) or SplitKV.auto()")
    ap.add_argument("--split-case", default="zipf", choices=["zipf", "hot"],
                    help="split workload lists: C5's Zipf(1.2) lengths, or 'hot' (H=8, 16 rows per head "
                         "select every block, the other rows 8 blocks)")
    ap.add_argument("--workload", default="echosparse", choices=["echosparse", "vsa", "vsa2_rep", "split"],
                    help="echosparse: the headline sparse step (default); vsa / vsa2_rep / split: the VSA "
                         "configurations (fine fwd+bwd at 30720 tokens, three-tier at the HunyuanVideo shape, "
                         "Zipf-skewed split-KV)")
    return ap.parse_args()


def executed_flops(ps, D=128):
    """4 * 128 * D * (64 * exact + means + 4 * refined), summed over (tile, head): one branch's sparse kernel."""
    cols = 64 * ps.counts.double().sum() + ps.mean_counts.double().sum() + 4 * ps.refine_counts.double().sum()
    return float(4 * 128 * D * cols)


def _host_cpu():
    """(CPU model string, os.cpu_count(), threads the CPU baseline uses). The threads are the host's CPU share for
    this job: OMP_NUM_THREADS when set (the GPU boxes set it to their per-GPU share, 16, whatever os.cpu_count()
    reports for the whole machine), else os.cpu_count()."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    count = os.cpu_count() or 1
    threads = int(os.environ.get("OMP_NUM_THREADS") or count)
    return model, count, max(1, min(threads, count))


def _timed_median(fn, runs=3):
    """Median wall time of `runs` calls of fn (after the caller's warm-up)."""
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def _cpu_threads(n):
    """Context that runs numpy's BLAS and torch's CPU ops on n threads."""
    from threadpoolctl import threadpool_limits
    torch.set_num_threads(n)
    return threadpool_limits(limits=n)


def cpu_baseline(q, k, v, attn, seconds):
    """The numpy oracle's fixed-offset sparse step on a bounded sample of (tile, head) pairs (head 0, first tiles),
    timed on this host with its CPU share of BLAS threads (median of 3 runs of about seconds / 3 each); returned
    as TFLOP/s on executed blocks, like `value`."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import echosparse_ref as ref
    ps, buf = attn._plan_scratch, attn._buffers
    st = attn._states[1]
    h = 0
    f = lambda x: x.float().cpu().numpy()
    qs, ks, vs = (f(x[:, h:h + 1]) for x in (q, k, v))
    comp = dict(k_mean=f(buf.k_mean[:, h:h + 1]), v_mean=f(buf.v_mean[:, h:h + 1]),
                means=ps.means[:, h:h + 1].cpu().numpy(), mean_counts=ps.mean_counts[:, h:h + 1].cpu().numpy(),
                refine=ps.refine[:, h:h + 1].cpu().numpy(), refine_counts=ps.refine_counts[:, h:h + 1].cpu().numpy(),
                k_rep=f(buf.reps.k[h:h + 1]), v_rep=f(buf.reps.v[h:h + 1]),
                log_counts=f(buf.reps.log_counts[h:h + 1]))
    counts, blocks = ps.counts[:, h:h + 1].cpu().numpy(), ps.blocks[:, h:h + 1].cpu().numpy()
    offset = f(st.offset(0)[:, h:h + 1])
    model, count, threads = _host_cpu()
    per_run = seconds / 3.0
    with _cpu_threads(threads):
        run = lambda n: ref.fixed_offset_attention(qs, ks, vs, counts, blocks, offset, comp=comp, tiles=n)
        run(1)                                                                              # warm-up
        tiles = 1
        while True:                                  # size the sample so that one run takes about seconds / 3
            t0 = time.perf_counter()
            run(tiles)
            elapsed = time.perf_counter() - t0
            if elapsed >= per_run or tiles >= counts.shape[0]:
                break
            tiles = min(counts.shape[0], max(tiles + 1, int(tiles * per_run / max(elapsed, 1e-3) * 1.05)))
        elapsed = _timed_median(lambda: run(tiles))
    cols = (64 * counts[:tiles].sum() + comp["mean_counts"][:tiles].sum() + 4 * comp["refine_counts"][:tiles].sum())
    flops = 4 * 128 * 128 * float(cols)
    return {"value": flops / elapsed / 1e12, "unit": "TFLOP/s (executed blocks)", "cores": threads,
            "os_cpu_count": count, "cpu_model": model, "kind": "port",
            "sample": f"numpy oracle fixed-offset sparse step (exact + mean + representative columns), head 0, query "
                      f"tiles 0..{tiles - 1} of {counts.shape[0]}, one branch; median of 3 runs, {elapsed:.1f} s "
                      f"each, {threads} BLAS threads",
            "ms_per_layer_extrapolated": elapsed / tiles * counts.shape[0] * q.shape[1] * 2 * 1e3}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py runs on one GPU only: the EchoSparse path shards by head with no exchange inside the "
              "attention, so this build measures one GPU's share; --gpus must be 1", file=sys.stderr)
        sys.exit(2)
    if args.workload != "echosparse":
        return run_vsa_workload(args)
    from self_trainable_or_free_attn_amd import EchoSparseAttention
    from self_trainable_or_free_attn_amd import synthetic
    from self_trainable_or_free_attn_amd.kernels import gfx950

    dev = torch.device("cuda:0")
    grid = tuple(int(x) for x in args.grid.split(","))
    H, D = args.heads, 128
    L = grid[0] * grid[1] * grid[2]
    t_setup = time.time()
    print(f"[bench] inputs grid={grid} L={L} H={H}", file=sys.stderr, flush=True)
    branches = []
    for b in range(2):        # two CFG branches: independent fields (seed per branch)
        q, k, v, _ = synthetic.fourier_qkv(grid, H, D, seed=11 + b, device=dev)
        prev = [synthetic.perturbed(x, 0.01, seed=100 + 10 * b + i) for i, x in enumerate((q, k, v))]
        branches.append(((q, k, v), prev))
    attn = EchoSparseAttention(density=args.density, dense_steps=2, dense_layers=())
    layer = 1
    # step 0: dense (offsets), step 1: full-block step (first map and plan), both on the perturbed inputs
    for step in range(2):
        for b in range(2):
            p = branches[b][1]
            attn(p[0][None], p[1][None], p[2][None], step, b, layer)
    torch.cuda.synchronize()
    print(f"[bench] setup {time.time() - t_setup:.1f}s", file=sys.stderr, flush=True)

    # time the dominant kernel with events on the stream it runs on (torch's current stream)
    K = attn.K
    orig = K.sparse_attention
    events = []

    def timed_sparse(*a, **kw):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        orig(*a, **kw)
        e1.record()
        events.append((e0, e1))

    K.sparse_attention = timed_sparse
    step = 2

    def one_layer(step):
        for b in range(2):
            c = branches[b][0]
            attn(c[0][None], c[1][None], c[2][None], step, b, layer)

    for _ in range(args.warmup):
        one_layer(step)
        step += 1
    torch.cuda.synchronize()
    events.clear()
    flops_steps = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_layer(step)
        step += 1
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    K.sparse_attention = orig
    ms_layer = elapsed / args.steps * 1e3
    kern_ms = sum(a.elapsed_time(b) for a, b in events) / max(1, len(events))
    ps = attn._plan_scratch
    fl_branch = executed_flops(ps, D)
    fl_layer = 2 * fl_branch
    value = fl_layer / (ms_layer * 1e-3) / 1e12
    achieved = fl_branch / (kern_ms * 1e-3) / 1e12
    nq, nb = -(-L // 128), -(-L // 64)
    mean_exact = float(ps.counts.double().mean())
    result = {
        "metric": "ms/layer + TFLOPS on executed blocks (% bf16 MFMA peak), Wan2.1-14B shape",
        "value": round(value, 2), "unit": "TFLOP/s (executed blocks, whole sparse-step layer)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_layer, 3),
        "ms_per_layer": round(ms_layer, 3), "pct_bf16_peak": round(100 * value * 1e12 / PEAK_BF16, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (Fourier-field Q/K, N(0,1) V, Morton order; random init, no checkpoint)",
        "config": {"workload": "echosparse_sparse_step_wan2.1_14b", "cfg_branches": 2, "heads": H, "seq_len": L,
                   "head_dim": D, "grid": list(grid), "density": args.density, "query_tiles": nq, "kv_blocks": nb,
                   "mean_exact_blocks_per_tile": round(mean_exact, 2),
                   "mean_mean_columns_per_tile": round(float(ps.mean_counts.double().mean()), 2),
                   "mean_refined_blocks_per_tile": round(float(ps.refine_counts.double().mean()), 2),
                   "executed_tflop_per_layer": round(fl_layer / 1e12, 3)},
        "roofline": {"kernel": "attn_kernel<FIXED,COMP,*> (es_sparse_attention, both CFG branches)", "bound": "mfma",
                     "achieved": round(achieved, 2), "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                     "frac": round(achieved * 1e12 / PEAK_BF16, 4), "traffic": TRAFFIC_BYTES,
                     "avg_launch_ms": round(kern_ms, 3), "launches": len(events),
                     "flop_per_launch": fl_branch},
    }
    if not args.no_dense:
        q, k, v = branches[0][0]
        qt, kt, vt = (x.permute(1, 0, 2)[None] for x in (q, k, v))
        for _ in range(2):
            torch.nn.functional.scaled_dot_product_attention(qt, kt, vt)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(3):
            torch.nn.functional.scaled_dot_product_attention(qt, kt, vt)
        torch.cuda.synchronize()
        sdpa_ms = (time.perf_counter() - t0) / 3 * 1e3
        gfx950.dense_attention(q, k, v)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(3):
            gfx950.dense_attention(q, k, v)
        torch.cuda.synchronize()
        own_ms = (time.perf_counter() - t0) / 3 * 1e3
        dense_flops = 4.0 * L * L * D * H
        result["dense"] = {"torch_sdpa_ms_per_layer": round(2 * sdpa_ms, 3),
                           "own_dense_ms_per_layer": round(2 * own_ms, 3),
                           "torch_sdpa_tflops": round(dense_flops / (sdpa_ms * 1e-3) / 1e12, 1),
                           "own_dense_tflops": round(dense_flops / (own_ms * 1e-3) / 1e12, 1),
                           "speedup_vs_sdpa": round(2 * sdpa_ms / ms_layer, 2)}
    if not args.no_cpu:
        c0, c1 = branches[0][0], None
        result["cpu_baseline"] = cpu_baseline(*c0, attn, args.cpu_seconds)
    print(json.dumps(result), flush=True)


# ------------------------------------------------------------------------------------------------ VSA workloads
def _timed(fn, steps, warmup):
    """(mean ms per call over `steps` calls after `warmup`, last result), bracketed by synchronisations."""
    out = None
    for _ in range(warmup):
        out = fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e3, out


def _events(fn, steps):
    """mean ms of fn measured with HIP events on torch's current stream (the stream every kernel here uses)."""
    ms = []
    for _ in range(steps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
    return sum(ms) / len(ms)


def _vsa_cpu_baseline(q, k, v, blk, sel, seconds):
    """The blockwise numpy port of the fine forward (oracle) on the first query blocks of head 0, sized so one run
    takes about seconds / 3; median of 3 runs on the host's CPU share of BLAS threads."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import vsa_ref as ref
    f = lambda x: x[0].float().cpu().numpy()
    qn, kn, vn = f(q), f(k), f(v)
    cnt = blk.cpu().numpy()
    ptr, idx = sel.q2k_ptr.cpu().numpy(), sel.q2k_idx.cpu().numpy()
    nb = cnt.size
    model, count, threads = _host_cpu()
    with _cpu_threads(threads):
        run = lambda n: ref.fine_attention_blocks(qn, kn, vn, cnt, ptr, idx, 0, list(range(n)))
        run(1)
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds / 3.0 and done < nb:
            ref.fine_attention_blocks(qn, kn, vn, cnt, ptr, idx, 0, [done])
            done += 1
        el = _timed_median(lambda: run(done))
    cols = int(ptr[0, 0, done] - ptr[0, 0, 0])
    flops = 4.0 * 64 * 64 * q.shape[-1] * cols
    return {"value": round(flops / el / 1e12, 5), "unit": "TFLOP/s (fine forward, executed blocks)",
            "cores": threads, "os_cpu_count": count, "cpu_model": model, "kind": "port",
            "sample": f"blockwise numpy port of the fine forward (oracle/vsa_ref.py fine_attention_blocks), head 0, "
                      f"query blocks 0..{done - 1} of {nb}, {cols} block pairs; median of 3 runs, {el:.1f} s each, "
                      f"{threads} BLAS threads"}


def run_vsa_workload(args):
    from self_trainable_or_free_attn_amd import synthetic
    from self_trainable_or_free_attn_amd.vsa import ops, rep
    dev = torch.device("cuda:0")
    W, K = max(1, args.warmup), max(1, args.steps)
    D = 128
    if args.workload in ("vsa", "split"):
        if args.workload == "vsa":   # C2: B1 H24 N30720, top-60 by the original-VSA router, N(0, 1) seed 1
            B, H, NB = 1, 24, 480
        elif args.split_case == "zipf":  # C5: B1 H40 L75648, Zipf(1.2) lists clipped to [8, 512], seed 4
            B, H, NB = 1, 40, 1182
        else:                        # hot rows: a few lists hold most of the work
            B, H, NB = 1, 8, 1182
        g = torch.Generator(device=dev).manual_seed(1 if args.workload == "vsa" else 4)
        q, k, v, dout = (torch.randn(B, H, NB * 64, D, device=dev, generator=g).to(torch.bfloat16) for _ in range(4))
        blk = torch.full((NB,), 64, dtype=torch.int32, device=dev)
        if args.workload == "vsa":
            sel = ops.route_rows(q, k, blk, 60)
        else:
            import numpy as np
            rng = np.random.default_rng(4)
            mask = np.zeros((B, H, NB, NB), bool)
            if args.split_case == "zipf":
                n = np.clip(rng.zipf(1.2, size=(B, H, NB)), 8, 512)
            else:
                n = np.full((B, H, NB), 8)
                n[:, :, rng.choice(NB, size=16, replace=False)] = NB
            for h in range(H):
                for i in range(NB):
                    mask[0, h, i, rng.choice(NB, size=int(n[0, h, i]), replace=False)] = True
            sel = ops.mask_to_selection(torch.as_tensor(mask, device=dev))
        nnz = int((sel.q2k_ptr[..., -1] - sel.q2k_ptr[..., 0]).sum())
        qg, kg, vg = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
        # C5: the manual policy (every list longer than 64 blocks runs as balanced 64-block chunks + ordered merge)
        split = None
        if args.workload == "split":
            split = ops.SplitKV.auto() if args.split_policy == "auto" else ops.SplitKV(chunk=64)

        def fwd():
            return ops.fine_block_sparse_attention(qg, kg, vg, blk, sel, split_kv=split)

        def fwd_bwd():
            o, _ = fwd()
            return torch.autograd.grad(o, (qg, kg, vg), dout)

        fwd_ms, _ = _timed(lambda: fwd(), K, W)
        step_ms, _ = _timed(fwd_bwd, K, W)
        fwd_ev = _events(lambda: fwd(), min(K, 5))
        fl_fwd = 4.0 * 64 * 64 * D * nnz
        fl_bwd = 14.0 * 64 * 64 * D * nnz    # KV-owner (4 products) + Q-owner (3 products) per pair
        res = {"metric": "ms/layer + TFLOPS on executed blocks (% bf16 MFMA peak), VSA fine attention fwd+bwd",
               "value": round((fl_fwd + fl_bwd) / (step_ms * 1e-3) / 1e12, 2),
               "unit": "TFLOP/s (executed blocks, fine fwd+bwd)", "n_gpus": 1, "steps": K, "warmup": W,
               "ms_per_step": round(step_ms, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
               "dtype": "bf16", "data": "synthetic (N(0,1) q/k/v/dO, seeded)",
               "config": {"workload": "vsa_c2_fine_fwd_bwd" if args.workload == "vsa" else
                          ("vsa_c5_zipf_split" if args.split_case == "zipf" else "vsa_hot_rows_split"),
                          "batch": B, "heads": H, "seq_len": NB * 64, "head_dim": D, "nnz_pairs": nnz,
                          "split_kv": None if split is None else
                          ("auto" if split.policy is not None else "manual chunk 64")},
               "fwd_ms": round(fwd_ms, 3), "bwd_ms": round(step_ms - fwd_ms, 3),
               "fwd_tflops": round(fl_fwd / (fwd_ms * 1e-3) / 1e12, 2),
               "roofline": {"kernel": "vsa_fwd_kernel (fine forward)", "bound": "mfma",
                            "achieved": round(fl_fwd / (fwd_ev * 1e-3) / 1e12, 2), "peak": PEAK_BF16 / 1e12,
                            "unit": "TFLOP/s", "frac": round(fl_fwd / (fwd_ev * 1e-3) / PEAK_BF16, 4),
                            "traffic": None, "avg_launch_ms": round(fwd_ev, 3)}}
        if args.workload == "split":
            unsplit_ms, _ = _timed(lambda: torch.autograd.grad(
                ops.fine_block_sparse_attention(qg, kg, vg, blk, sel)[0], (qg, kg, vg), dout), K, W)
            res["unsplit_ms_per_step"] = round(unsplit_ms, 3)
            res["split_speedup"] = round(unsplit_ms / step_ms, 3)
            plan = ops.describe_split(qg, sel, split)
            res["split_plan"] = {d: plan[d]["info"] for d in plan}
        if not args.no_cpu:
            res["cpu_baseline"] = _vsa_cpu_baseline(q, k, v, blk, sel, args.cpu_seconds)
        print(json.dumps(res), flush=True)
        return
    # C4: VSA2 three-tier at the HunyuanVideo shape: B2 H24, 33 x 45 x 80 grid (118800 tokens, 1857 blocks),
    # Fourier-field Q / K, N(0, 1) V; tiers 5 % full, 20 % x 4 representatives, the rest block means
    grid = (33, 45, 80)
    Lr = grid[0] * grid[1] * grid[2]
    NB = -(-Lr // 64)
    B, H = 2, 24
    xs = []
    for b in range(B):
        qb, kb, vb, _ = synthetic.fourier_qkv(grid, H, D, seed=21 + b, device=dev, pad_to=NB * 64)
        xs.append([t.permute(1, 0, 2) for t in (qb, kb, vb)])
    q, k, v = (torch.stack([x[i] for x in xs]).contiguous() for i in range(3))
    del xs
    blk = torch.full((NB,), 64, dtype=torch.int32, device=dev)
    blk[-1] = Lr - 64 * (NB - 1)
    g = torch.Generator(device=dev).manual_seed(5)
    dout = torch.randn(q.shape, device=dev, generator=g).to(torch.bfloat16)
    baseline = args.c4 == "baseline"
    tiers = rep.RepTiers(frac_full=0.05, frac_mid=0.20, mid_reps=4, split="per_row" if baseline else "global",
                         tables="kmeans" if baseline else "contiguous", kmeans_iters=5, seed=0)
    sel = rep.route_tiers(q, k, blk, tiers, R=16)
    a, b, c = sel.tier_masks(NB)
    na, nbm, ncm = (int(m.sum()) for m in (a, b, c))
    cols = 64 * na + 4 * nbm + ncm                 # columns over all (b, h, query block)
    fl_fwd = 4.0 * 64 * D * cols
    qg, kg, vg = (x.detach().clone().requires_grad_(True) for x in (q, k, v))

    def fwd():   # (the representative tables are built inside, k-means included)
        return rep.rep_fine_attention(qg, kg, vg, blk, sel, mid_reps=4, tables=tiers.tables,
                                      kmeans_iters=tiers.kmeans_iters, seed=tiers.seed)

    def fwd_bwd():
        o, _ = fwd()
        return torch.autograd.grad(o, (qg, kg, vg), dout)

    fwd_ms, _ = _timed(fwd, K, W)
    step_ms, _ = _timed(fwd_bwd, K, W)
    route_ms, _ = _timed(lambda: rep.route_tiers(q, k, blk, tiers, R=16), min(K, 3), 1)
    tables_ms, _ = _timed(lambda: rep.build_tables(k, v, blk, rep._Tables.of(tiers)), min(K, 3), 1)
    fwd_ev = _events(fwd, min(K, 5))
    res = {"metric": "ms/layer + TFLOPS on executed blocks (% bf16 MFMA peak), VSA2 64/4/1 three-tier fine fwd+bwd",
           "value": round(fl_fwd / (fwd_ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s (executed columns, fine forward)",
           "n_gpus": 1, "steps": K, "warmup": W, "ms_per_step": round(step_ms, 3), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic (Fourier-field Q/K, N(0,1) V and dO, Morton order; seeded)",
           "config": {"workload": "vsa2_rep_c4_hunyuan", "construction": args.c4, "split": tiers.split,
                      "tables": tiers.tables, "batch": B, "heads": H, "seq_len": NB * 64,
                      "valid_tokens": Lr, "head_dim": D, "tier_pairs": {"A": na, "B": nbm, "C": ncm},
                      "columns_per_query_block": round(cols / (B * H * NB), 1)},
           "fwd_ms": round(fwd_ms, 3), "bwd_ms": round(step_ms - fwd_ms, 3), "route_tiers_ms": round(route_ms, 3),
           "tables_ms_in_fwd": round(tables_ms, 3),
           "roofline": {"kernel": "rep_q_kernel<false> (three-tier forward)", "bound": "mfma",
                        "achieved": round(fl_fwd / (fwd_ev * 1e-3) / 1e12, 2), "peak": PEAK_BF16 / 1e12,
                        "unit": "TFLOP/s", "frac": round(fl_fwd / (fwd_ev * 1e-3) / PEAK_BF16, 4), "traffic": None,
                        "avg_launch_ms": round(fwd_ev, 3)}}
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
