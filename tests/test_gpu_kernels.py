"""Parity of every gfx950 kernel of the EchoSparse set with the CPU oracle (oracle/echosparse_ref.py), through the
C ABI (the kernels.gfx950 wrappers are thin calls of its torch operators, torch.ops.echosparse_gfx950). Floating-point outputs: max-abs 2e-2 and rel-L2 1e-2;
plan outputs (keep, lists, counts, bit masks): bit-exact. Shapes follow the reference's own GPU tests
(L = 4152: 65 kv blocks with a 56-token tail, 33 query tiles with a 56-row tail)."""
import math
import sys

import numpy as np
import pytest
import torch

from helpers import check_close, f32, structured_qkv
from oracle import echosparse_ref as ref

pytestmark = pytest.mark.gpu

L, H, D = 4152, 2, 128
NQ, NB = ref.cdiv(L, 128), ref.cdiv(L, 64)


def K():
    from self_trainable_or_free_attn_amd.kernels import gfx950
    return gfx950


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def data(dev):
    (q, k, v), = structured_qkv(L, H, seed=0)
    return dict(q=q, k=k, v=v, qd=q.to(dev), kd=k.to(dev), vd=v.to(dev))


@pytest.fixture(scope="module")
def dense(data):
    """Oracle dense log2 LSE (prior for later tests), in the offset layout."""
    nq = NQ
    off = np.full((nq * 128, H), 1e30, np.float32)
    allb = np.broadcast_to(np.arange(NB, dtype=np.int32), (nq, H, NB))
    cnt = np.full((nq, H), NB, np.int32)
    out, lse, _, _ = ref.fixed_offset_attention(f32(data["q"]), f32(data["k"]), f32(data["v"]), cnt, allb,
                                                np.zeros((nq * 128, H), np.float32))
    lse = lse.astype(np.float32)
    lse[L:] = 1e30
    return out, lse


def test_library_loads_and_reports_errors(dev):
    from self_trainable_or_free_attn_amd import _lib
    assert _lib.lib().es_abi_version() == _lib.ABI_VERSION == 2
    q = torch.zeros(64, 1, 64, device=dev, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="head dimension must be 128"):
        _lib.call("es_block_means", q, q, q, q, 64, 1, 64)


def test_torch_operators_refuse_views_wrong_dtypes_and_wrapping_ints(data):
    """The generated operators check every tensor's layout and dtype against the C type and every int against its
    C range before the launch, so a strided view or an fp32 tensor where bf16 is expected never reaches a kernel."""
    ops = torch.ops.echosparse_gfx950
    kd, vd = data["kd"], data["vd"]
    km = torch.zeros(NB, H, D, device=kd.device, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="argument k must be contiguous"):
        ops.es_block_means(kd.transpose(0, 1), vd, km, km.clone(), L, H, D)
    with pytest.raises(RuntimeError, match="argument v must be bfloat16 or float16"):
        ops.es_block_means(kd, vd.float(), km, km.clone(), L, H, D)
    with pytest.raises(RuntimeError, match="argument L = 4294967360 is out of range"):
        ops.es_block_means(kd, vd, km, km.clone(), 2 ** 32 + 64, H, D)
    cnt = torch.zeros(NQ, H, device=kd.device, dtype=torch.int64)
    lse = torch.zeros(NQ * 128, H, device=kd.device)
    with pytest.raises(RuntimeError, match="argument counts must be int32"):
        ops.es_exact_fallback(data["qd"], kd, vd, torch.empty_like(data["qd"]), cnt, cnt.int(), NB, lse,
                              cnt.int(), L, H, D)
    torch.cuda.synchronize()


def test_balanced_launch_replays_in_a_graph(data):
    """A balanced launch (dense attention) captured in a HIP graph takes its counter slot from the captured ring:
    three replays, with uncaptured launches of the same kernel and host synchronisations between them, each write
    the eager bytes."""
    qd, kd, vd = data["qd"], data["kd"], data["vd"]
    ops = torch.ops.echosparse_gfx950
    out_e = torch.empty_like(qd)
    lse_e = torch.empty(NQ * 128, H, device=qd.device)
    ops.es_dense_attention(qd, kd, vd, out_e, lse_e, L, H, D)
    torch.cuda.synchronize()
    out_g = torch.zeros_like(qd)
    lse_g = torch.zeros_like(lse_e)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ops.es_dense_attention(qd, kd, vd, out_g, lse_g, L, H, D)
    torch.cuda.synchronize()
    for rep in range(3):
        log("graph replay", rep)
        out_g.zero_()
        lse_g.zero_()
        g.replay()
        other_o, other_l = torch.empty_like(qd), torch.empty_like(lse_e)
        ops.es_dense_attention(qd, kd, vd, other_o, other_l, L, H, D)
        torch.cuda.synchronize()
        assert torch.equal(out_g.view(torch.int16), out_e.view(torch.int16)), rep
        assert torch.equal(lse_g, lse_e), rep
        assert torch.equal(other_o.view(torch.int16), out_e.view(torch.int16)), rep


def test_torch_operator_matches_the_direct_c_call_and_compiles(data):
    """The torch operator and a direct ctypes call of the same entry point write the same bytes; under
    torch.compile (AOT autograd: functionalisation of the declared writes, fake tensors through the Meta kernel)
    the compiled function returns the eager result."""
    import ctypes
    from self_trainable_or_free_attn_amd import _lib
    kd, vd = data["kd"], data["vd"]
    a = [torch.full((NB, H, D), 7.0, device=kd.device, dtype=torch.bfloat16) for _ in range(4)]
    _lib.ops().es_block_means(kd, vd, a[0], a[1], L, H, D)
    st = _lib.lib().es_block_means(_lib.ptr(kd), _lib.ptr(vd), _lib.ptr(a[2]), _lib.ptr(a[3]), L, H, D,
                                   ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0
    torch.cuda.synchronize()
    assert torch.equal(a[0].view(torch.int16), a[2].view(torch.int16))
    assert torch.equal(a[1].view(torch.int16), a[3].view(torch.int16))

    def f(k, v):
        km = torch.zeros(NB, H, D, device=k.device, dtype=torch.bfloat16)
        vm = torch.zeros_like(km)
        torch.ops.echosparse_gfx950.es_block_means(k, v, km, vm, L, H, D)
        return km.float() * 2.0 + vm.float()

    log("torch.compile(aot_eager) of es_block_means")
    got = torch.compile(f, backend="aot_eager", fullgraph=True)(kd, vd)
    torch.cuda.synchronize()
    assert torch.equal(got, a[0].float() * 2.0 + a[1].float())


def test_dense_attention(data, dense):
    log("dense attention L", L, "H", H)
    out, lse2 = K().dense_attention(data["qd"], data["kd"], data["vd"])
    torch.cuda.synchronize()
    ro, rl = dense
    check_close("dense O", f32(out), ro)
    check_close("dense LSE", f32(lse2)[:L], rl[:L])
    assert (f32(lse2)[L:] == 1e30).all()


def test_block_means(data):
    km = torch.empty(NB, H, D, device=data["kd"].device, dtype=torch.bfloat16)
    vm = torch.empty_like(km)
    K().block_means(data["kd"], data["vd"], km, vm)
    rk, rv = ref.block_means(f32(data["k"]), f32(data["v"]))
    # fp32 sums in another order than the float64 oracle: at most one bf16 ulp apart
    for got, want in ((f32(km), rk), (f32(vm), rv)):
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -14))) - 7)
        assert (np.abs(got - want) <= ulp).all()


def test_full_step_block_attention(data, dense):
    """All blocks at the fixed offset (prior = the dense LSE): O equals dense attention, the row sums are ~1 so no
    tile flags, LSE = prior + log2(sum), and the map is the per-block probability mass."""
    dev = data["qd"].device
    prior = dense[1] + 0.1 * np.sin(np.arange(NQ * 128))[:, None].astype(np.float32)
    prior[L:] = 1e30
    offset = torch.from_numpy(prior).to(dev)
    allb = torch.arange(NB, device=dev, dtype=torch.int32).expand(NQ, H, NB).contiguous()
    cnt = torch.full((NQ, H), NB, device=dev, dtype=torch.int32)
    out = torch.empty_like(data["qd"])
    lse = torch.empty(NQ * 128, H, device=dev)
    flags = torch.full((NQ, H), 7, device=dev, dtype=torch.int32)
    mass = torch.zeros(H, NQ, NB, device=dev)
    K().block_attention(data["qd"], data["kd"], data["vd"], out, cnt, allb, offset, lse, flags, mass=mass)
    torch.cuda.synchronize()
    ro, rl, rf, rm = ref.fixed_offset_attention(f32(data["q"]), f32(data["k"]), f32(data["v"]), cnt.cpu().numpy(),
                                                allb.cpu().numpy(), prior, write_mass=True)
    check_close("full O", f32(out), ro)
    check_close("full LSE", f32(lse)[:L], rl[:L])
    assert (f32(lse)[L:] == 1e30).all()
    assert np.array_equal(flags.cpu().numpy(), rf) and rf.sum() == 0
    check_close("full mass", f32(mass), rm, max_abs=2e-2 * max(1.0, float(np.abs(rm).max())))


@pytest.fixture(scope="module")
def plan(data, dense):
    """A sparse-step plan from the oracle: full-step map at the dense prior -> select -> pack -> rebuild."""
    prior = dense[1]
    allb = np.broadcast_to(np.arange(NB, dtype=np.int32), (NQ, H, NB))
    cnt = np.full((NQ, H), NB, np.int32)
    _, lse, flags, mass = ref.fixed_offset_attention(f32(data["q"]), f32(data["k"]), f32(data["v"]), cnt, allb,
                                                     prior, write_mass=True)
    lse = lse.astype(np.float32)
    se, ss = ref.full_step_scales(prior, lse, L)
    top, refined = ref.budget(0.1, NB)
    rw = -(-refined // 32) * 32
    words = ref.plan_words(NB)
    keep, counts, blocks, refine, skip = ref.select_blocks(
        mass.astype(np.float32), np.ones((H, NQ, NB), np.uint8), se.astype(np.float32), ss.astype(np.float32),
        flags, top, refined, L, rw, words)
    exact = ref.pack_plan(keep, words)
    lists = ref.rebuild_plan(exact, skip, NB, rw)
    return dict(prior=prior, mass=mass.astype(np.float32), lse=lse, se=se.astype(np.float32),
                ss=ss.astype(np.float32), flags=flags, top=top, refined=refined, rw=rw, words=words, keep=keep,
                counts=counts, blocks=blocks, refine=refine, skip=skip, exact=exact, lists=lists)


def test_select_blocks_bit_exact(plan, dev):
    p = plan
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    keep = torch.full((H, NQ, NB), 7, device=dev, dtype=torch.uint8)
    counts = torch.full((NQ, H), 7, device=dev, dtype=torch.int32)
    blocks = torch.zeros(NQ, H, NB, device=dev, dtype=torch.int32)
    skip = torch.full((H, NQ, p["words"]), -1, device=dev, dtype=torch.int32)
    refine = torch.full((NQ, H, p["rw"]), 7, device=dev, dtype=torch.int32)
    K().select_blocks(t(p["mass"]), t(np.ones((H, NQ, NB), np.uint8)), t(p["se"]), t(p["ss"]), keep, counts, blocks,
                      t(p["flags"]), skip, refine, p["top"], p["refined"], L)
    torch.cuda.synchronize()
    assert np.array_equal(keep.cpu().numpy(), p["keep"])
    assert np.array_equal(counts.cpu().numpy(), p["counts"])
    used = np.arange(NB)[None, None, :] < p["counts"][..., None]
    assert np.array_equal(blocks.cpu().numpy()[used], p["blocks"][used])
    assert np.array_equal(refine.cpu().numpy(), p["refine"])
    assert np.array_equal(skip.cpu().numpy(), p["skip"])


@pytest.mark.parametrize("case", ["ties", "sink_flags_nan"])
def test_select_blocks_edge_cases(case, dev):
    """Hand-made maps: many equal values around the K-th (threshold inclusion keeps all ties), refine index cut,
    a sink, fell-back tiles and NaN entries."""
    g = np.random.default_rng(3)
    mass = g.integers(0, 5, size=(H, NQ, NB)).astype(np.float32) / 4
    keep_prev = (g.random((H, NQ, NB)) < 0.2).astype(np.uint8)
    se = np.full((H, NQ), 1.0, np.float32)
    ss = np.full((H, NQ), 0.5, np.float32)
    flags = np.zeros((NQ, H), np.int32)
    sink = 1 << 30
    if case == "sink_flags_nan":
        mass[g.random(mass.shape) < 0.05] = np.nan
        flags[::3] = 1
        sink = 60
        se = g.random((H, NQ)).astype(np.float32) + 0.5
    top, refined = 7, 20
    rw, words = 32, ref.plan_words(NB)
    r = ref.select_blocks(mass, keep_prev, se, ss, flags, top, refined, L, rw, words, sink=sink)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    keep = torch.empty(H, NQ, NB, device=dev, dtype=torch.uint8)
    counts = torch.empty(NQ, H, device=dev, dtype=torch.int32)
    blocks = torch.zeros(NQ, H, NB, device=dev, dtype=torch.int32)
    skip = torch.full((H, NQ, words), -1, device=dev, dtype=torch.int32)
    refine = torch.empty(NQ, H, rw, device=dev, dtype=torch.int32)
    K().select_blocks(t(mass), t(keep_prev), t(se), t(ss), keep, counts, blocks, t(flags), skip, refine, top,
                      refined, L, sink=sink)
    torch.cuda.synchronize()
    assert np.array_equal(keep.cpu().numpy(), r[0])
    assert np.array_equal(counts.cpu().numpy(), r[1])
    used = np.arange(NB)[None, None, :] < r[1][..., None]
    assert np.array_equal(blocks.cpu().numpy()[used], r[2][used])
    assert np.array_equal(refine.cpu().numpy(), r[3])
    assert np.array_equal(skip.cpu().numpy(), r[4])


def test_pack_plan_bit_order_known_value(dev):
    """The kernel's plan word layout against a literal: nb = 40 with blocks 0, 5 and 33 kept packs to 0x21,
    0xFFFFFF02 (bit i of word w = block 32 w + i, blocks 40..63 set); rebuilding lists exactly those blocks."""
    keep = torch.zeros(1, 1, 40, device=dev, dtype=torch.uint8)
    keep[0, 0, [0, 5, 33]] = 1
    exact = torch.full((1, 1, 4), -1, device=dev, dtype=torch.int32)
    K().pack_plan(keep, exact)
    torch.cuda.synchronize()
    assert exact.cpu().tolist() == [[[0x21, -254, -1, -1]]]


def test_pack_and_rebuild_bit_exact(plan, dev):
    p = plan
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    exact = torch.full((H, NQ, p["words"]), 5, device=dev, dtype=torch.int32)
    K().pack_plan(t(p["keep"]), exact)
    torch.cuda.synchronize()
    assert np.array_equal(exact.cpu().numpy(), p["exact"])
    keep = torch.full((H, NQ, NB), 7, device=dev, dtype=torch.uint8)
    counts, rc, mc = (torch.full((NQ, H), 7, device=dev, dtype=torch.int32) for _ in range(3))
    blocks, means = (torch.zeros(NQ, H, NB, device=dev, dtype=torch.int32) for _ in range(2))
    refine = torch.full((NQ, H, p["rw"]), 7, device=dev, dtype=torch.int32)
    K().rebuild_plan(t(p["exact"]), t(p["skip"]), keep, counts, blocks, refine, rc, means, mc)
    torch.cuda.synchronize()
    rk, rcnt, rblocks, rref, rrc, rmeans, rmc = p["lists"]
    assert np.array_equal(keep.cpu().numpy(), rk) and np.array_equal(rk, p["keep"])
    assert np.array_equal(counts.cpu().numpy(), rcnt)
    used = np.arange(NB)[None, None, :] < rcnt[..., None]
    assert np.array_equal(blocks.cpu().numpy()[used], rblocks[used])
    assert np.array_equal(refine.cpu().numpy(), rref) and np.array_equal(rref, p["refine"])
    assert np.array_equal(rc.cpu().numpy(), rrc)
    assert np.array_equal(mc.cpu().numpy(), rmc)
    usedm = np.arange(NB)[None, None, :] < rmc[..., None]
    assert np.array_equal(means.cpu().numpy()[usedm], rmeans[usedm])


@pytest.fixture(scope="module")
def reps(data):
    dev = data["qd"].device
    R = K().Representatives(L, H, D, dev, iters=6)
    km = torch.empty(NB, H, D, device=dev, dtype=torch.bfloat16)
    vm = torch.empty_like(km)
    R.build(data["qd"], data["kd"], data["vd"], km, vm)
    torch.cuda.synchronize()
    return R, km, vm


def test_representatives_invariants(data, reps):
    """Counts sum to the block length and the count-weighted representatives add up to the block sum (reference
    tests/test_sm120.py:65-83); the fused block means equal the block_means kernel byte for byte; the sentinel
    block stays empty."""
    R, km, vm = reps
    km2, vm2 = torch.empty_like(km), torch.empty_like(vm)
    K().block_means(data["kd"], data["vd"], km2, vm2)
    torch.cuda.synchronize()
    assert torch.equal(km.view(torch.int16), km2.view(torch.int16)) and torch.equal(vm.view(torch.int16),
                                                                                     vm2.view(torch.int16))
    lc = f32(R.log_counts)
    counts = np.exp2(lc[:, :4 * NB]).reshape(H, NB, 4)
    sizes = np.full(NB, 64.0)
    sizes[-1] = L - 64 * (NB - 1)
    assert np.allclose(counts.sum(-1), sizes[None, :], atol=1e-3)
    for rep, x in ((R.k, data["k"]), (R.v, data["v"])):
        total = (f32(rep)[:, :4 * NB].reshape(H, NB, 4, D) * counts[..., None]).sum(2)
        xs = np.concatenate([f32(x), np.zeros((NB * 64 - L, H, D), np.float32)]).reshape(NB, 64, H, D).sum(1)
        want = xs.transpose(1, 0, 2)
        assert np.linalg.norm(total - want) / np.linalg.norm(want) < 1e-2
    assert (f32(R.k)[:, 4 * NB:] == 0).all() and np.isneginf(lc[:, 4 * NB:]).all()


def test_representatives_match_oracle(data, reps):
    """The clustering decisions match the oracle on almost every block (float rounding can flip a token that sits
    on a cluster boundary), and the representatives of matching blocks agree at tolerance."""
    R, _, _ = reps
    rk, rv, rl = ref.representatives(f32(data["q"]), f32(data["k"]), f32(data["v"]), iters=6)
    lc = f32(R.log_counts)
    same = (np.isclose(lc, rl) | (np.isneginf(lc) & np.isneginf(rl)))[:, :4 * NB].reshape(H, NB, 4).all(-1)
    log("blocks with identical cluster sizes:", same.mean())
    assert same.mean() > 0.9
    gk = f32(R.k)[:, :4 * NB].reshape(H, NB, 4, D)[same]
    wk = rk[:, :4 * NB].reshape(H, NB, 4, D)[same]
    # blocks with the oracle's cluster sizes hold the same members: the bf16 means of the same tokens (flat bounds)
    log("rep k max-abs / rel-L2", *check_close("rep k", gk, wk))


def test_sparse_attention(data, plan, reps, dev):
    """The sparse step's fixed-offset kernel with compensation columns, against the oracle fed the same plan,
    block means and representatives; `mass` holds the exact blocks' masses."""
    p = plan
    R, km, vm = reps
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    keep, counts, blocks, refine, rc, means, mc = (t(x) for x in p["lists"])
    offset = t(p["lse"])
    out = torch.full_like(data["qd"], 7.0)
    lse = torch.full((NQ * 128, H), 7.0, device=dev)
    flags = torch.full((NQ, H), 7, device=dev, dtype=torch.int32)
    mass = torch.zeros(H, NQ, NB, device=dev)
    K().sparse_attention(data["qd"], data["kd"], data["vd"], km, vm, means, mc, out, counts, blocks, offset, lse,
                         flags, refine, rc, R.k, R.v, R.log_counts, mass=mass)
    torch.cuda.synchronize()
    comp = dict(k_mean=f32(km), v_mean=f32(vm), means=p["lists"][5], mean_counts=p["lists"][6],
                refine=p["lists"][3], refine_counts=p["lists"][4], k_rep=f32(R.k), v_rep=f32(R.v),
                log_counts=f32(R.log_counts))
    ro, rl, rf, rm = ref.fixed_offset_attention(f32(data["q"]), f32(data["k"]), f32(data["v"]), p["lists"][1],
                                                p["lists"][2], p["lse"], comp=comp, write_mass=True)
    check_close("sparse O", f32(out), ro)
    check_close("sparse LSE", f32(lse)[:L], rl[:L])
    assert (f32(lse)[L:] == 1e30).all()
    assert np.array_equal(flags.cpu().numpy(), rf)
    ex = p["lists"][0].astype(bool)
    check_close("sparse mass", f32(mass)[ex], rm[ex], max_abs=2e-2 * max(1.0, float(np.abs(rm).max())))
    assert (f32(mass)[~ex] == 0).all()


def test_estimate_and_scales(data, plan, reps, dev):
    p = plan
    R, km, vm = reps
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    g = np.random.default_rng(1)
    new_lse = p["lse"] + (g.standard_normal(p["lse"].shape) * 0.05).astype(np.float32)
    new_lse[L:] = 1e30
    mass0 = np.where(p["keep"] != 0, p["mass"], 0).astype(np.float32)
    mass = t(mass0)
    se = torch.empty(H, NQ, device=dev)
    ss = torch.empty(H, NQ, device=dev)
    K().estimate_skipped(data["qd"], km, t(p["keep"]), t(p["lse"]), t(new_lse), mass, se, ss)
    torch.cuda.synchronize()
    rm = mass0.copy()
    rse, rss = ref.estimate_skipped(f32(data["q"]), f32(km), p["keep"], p["lse"], new_lse, rm)
    check_close("estimate map", f32(mass), rm, max_abs=2e-2 * max(1.0, float(np.abs(rm).max())))
    check_close("scale_exact", f32(se), rse)
    check_close("scale_skip", f32(ss), rss, max_abs=2e-2 * max(1.0, float(np.abs(rss).max())))
    # full-step scales
    lse2 = t(new_lse)
    lse2[L:] = 3.0
    se2 = torch.empty(H, NQ, device=dev)
    ss2 = torch.empty(H, NQ, device=dev)
    K().full_step_scales(t(p["lse"]), lse2, se2, ss2, L)
    torch.cuda.synchronize()
    rl = new_lse.copy()
    rse2, rss2 = ref.full_step_scales(p["lse"], rl, L)
    check_close("full scale_exact", f32(se2), rse2)
    assert (f32(ss2) == 1).all() and (f32(lse2)[L:] == 1e30).all()


def test_fallback_and_compensation(data, plan, reps, dev):
    """Every tile flagged (offset shifted by +200 as the reference's fallback test does): online softmax over the
    block list, then block-mean compensation of the keep == 0 blocks at the new LSE."""
    p = plan
    R, km, vm = reps
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    keep, counts, blocks = (t(x) for x in p["lists"][:3])
    out = torch.full_like(data["qd"], 3.0)
    lse = torch.full((NQ * 128, H), 5.0, device=dev)
    flags = torch.ones(NQ, H, device=dev, dtype=torch.int32)
    flags[0, 0] = 0
    K().exact_fallback(data["qd"], data["kd"], data["vd"], out, counts, blocks, lse, flags)
    torch.cuda.synchronize()
    ro = np.full((L, H, D), 3.0)
    rl = np.full((NQ * 128, H), 5.0)
    fl = flags.cpu().numpy()
    ref.exact_fallback(f32(data["q"]), f32(data["k"]), f32(data["v"]), ro, p["lists"][1], p["lists"][2], rl, fl)
    check_close("fallback O", f32(out), ro)
    check_close("fallback LSE", f32(lse)[:L], rl[:L])
    K().compensate_fallback(data["qd"], km, vm, keep, lse, out, flags)
    torch.cuda.synchronize()
    ref.compensate_fallback(f32(data["q"]), f32(km), f32(vm), p["lists"][0], rl, ro, fl)
    check_close("compensated O", f32(out), ro)
    check_close("compensated LSE", f32(lse)[:L], rl[:L])


def test_sparse_attention_stream_edges(data, plan, reps, dev):
    """Column streams that start with representative or mean chunks, a stream of 65 exact blocks (mass flush
    after block 63 and at the end), one chunk of each kind, unsorted exact lists with the partial tail block first
    or in the middle, lists of 4 and 5 exact blocks, against the oracle on the same lists: exercises the kernel's
    staged list ring, its first-chunk bias paths and the bounds of its exact-stretch loop."""
    p = plan
    R, km, vm = reps
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    keep, counts, blocks, refine, rc, means, mc = (np.array(x, copy=True) for x in p["lists"])
    counts[0, 0], mc[0, 0], rc[0, 0] = 0, 0, 3            # representatives only
    refine[0, 0, :3] = [3, 10, NB - 1]
    counts[1, 0], mc[1, 0], rc[1, 0] = 0, NB, 0           # block means only, two chunks
    means[1, 0, :NB] = np.arange(NB)
    counts[2, 0], mc[2, 0], rc[2, 0] = NB, 0, 0           # every block exact
    blocks[2, 0, :NB] = np.arange(NB)
    counts[3, 1], mc[3, 1], rc[3, 1] = 1, 1, 1            # one chunk of each kind, the tail block exact
    blocks[3, 1, 0], means[3, 1, 0], refine[3, 1, 0] = NB - 1, 0, 2
    # unsorted lists around the kernel's exact-stretch loop (chunks j .. j + 3 exact, chunk j not the tail block):
    # every block in descending order (the partial tail block first), the tail block in the middle of a list, and
    # lists of exactly 4 and 5 blocks
    counts[4, 0] = NB
    blocks[4, 0, :NB] = np.arange(NB)[::-1]
    counts[5, 1] = 20
    blocks[5, 1, :20] = [3, 10, 17, 24, 31, 38, 45, NB - 1, 1, 12, 23, 34, 56, 14, 25, 36, 47, 58, 0, 2]
    counts[6, 0] = 4
    blocks[6, 0, :4] = [0, 5, 9, NB - 1]
    counts[7, 1] = 5
    blocks[7, 1, :5] = [NB - 1, 2, 30, 31, 40]
    offset = t(p["lse"])
    out = torch.full_like(data["qd"], 7.0)
    lse = torch.full((NQ * 128, H), 7.0, device=dev)
    flags = torch.full((NQ, H), 7, device=dev, dtype=torch.int32)
    mass = torch.zeros(H, NQ, NB, device=dev)
    K().sparse_attention(data["qd"], data["kd"], data["vd"], km, vm, t(means), t(mc), out, t(counts), t(blocks),
                         offset, lse, flags, t(refine), t(rc), R.k, R.v, R.log_counts, mass=mass)
    torch.cuda.synchronize()
    comp = dict(k_mean=f32(km), v_mean=f32(vm), means=means, mean_counts=mc, refine=refine, refine_counts=rc,
                k_rep=f32(R.k), v_rep=f32(R.v), log_counts=f32(R.log_counts))
    ro, rl, rf, rm = ref.fixed_offset_attention(f32(data["q"]), f32(data["k"]), f32(data["v"]), counts, blocks,
                                                p["lse"], comp=comp, write_mass=True)
    check_close("edge O", f32(out), ro)
    check_close("edge LSE", f32(lse)[:L], rl[:L])
    assert np.array_equal(flags.cpu().numpy(), rf)
    ex = np.zeros((H, NQ, NB), bool)
    for qt in range(NQ):
        for hh in range(H):
            ex[hh, qt, blocks[qt, hh, :counts[qt, hh]]] = True
    check_close("edge mass", f32(mass)[ex], rm[ex], max_abs=2e-2 * max(1.0, float(np.abs(rm).max())))
    assert (f32(mass)[~ex] == 0).all()


def test_sparse_attention_balanced_launches_concurrent_and_repeated(data, plan, reps, dev):
    """The sparse step hands the last tiles of each XCD queue out at run time through a 64-slot ring of counters:
    launches on three streams at once and 70 launches in a row (the ring wraps) give bytes-identical outputs,
    which also pins that every tile runs exactly once whichever workgroup takes it."""
    p = plan
    R, km, vm = reps
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    keep, counts, blocks, refine, rc, means, mc = (t(x) for x in p["lists"])
    offset = t(p["lse"])

    def outputs():
        return (torch.full_like(data["qd"], 7.0), torch.full((NQ * 128, H), 7.0, device=dev),
                torch.full((NQ, H), 7, device=dev, dtype=torch.int32), torch.zeros(H, NQ, NB, device=dev))

    def call(o):
        K().sparse_attention(data["qd"], data["kd"], data["vd"], km, vm, means, mc, o[0], counts, blocks, offset,
                             o[1], o[2], refine, rc, R.k, R.v, R.log_counts, mass=o[3])

    want = outputs()
    call(want)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(3)]
    got = [outputs() for _ in streams]
    torch.cuda.synchronize()
    for s, o in zip(streams, got):
        with torch.cuda.stream(s):
            for _ in range(4):
                call(o)
    torch.cuda.synchronize()
    seq = outputs()
    for _ in range(70):
        call(seq)
    torch.cuda.synchronize()
    for o in got + [seq]:
        for a, b in zip(o, want):
            assert torch.equal(a, b)


def test_balanced_ring_waits_for_a_live_slot(data, plan, reps, dev):
    """A long balanced launch (dense attention, L = 32768, H = 8) on one stream while 70 short sparse launches run
    on another: the short ones wrap the 64-slot counter ring and reach the slot the long launch still uses; the
    launch that takes it must wait for the long one instead of clearing its counters, so every output is
    bytes-identical to the same launches run one after another."""
    p = plan
    R, km, vm = reps
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    keep, counts, blocks, refine, rc, means, mc = (t(x) for x in p["lists"])
    offset = t(p["lse"])
    g = torch.Generator(device=dev).manual_seed(11)
    Lb, Hb = 32768, 8
    qb, kb, vb = (torch.randn(Lb, Hb, D, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))

    def short(o):
        K().sparse_attention(data["qd"], data["kd"], data["vd"], km, vm, means, mc, o[0], counts, blocks, offset,
                             o[1], o[2], refine, rc, R.k, R.v, R.log_counts, mass=o[3])

    def outputs():
        return (torch.full_like(data["qd"], 7.0), torch.full((NQ * 128, H), 7.0, device=dev),
                torch.full((NQ, H), 7, device=dev, dtype=torch.int32), torch.zeros(H, NQ, NB, device=dev))

    log("ring: serial reference launches")
    want_long = K().dense_attention(qb, kb, vb)
    want = outputs()
    short(want)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    got = [outputs() for _ in range(70)]
    torch.cuda.synchronize()
    log("ring: long launch on stream A, 70 short launches on stream B")
    with torch.cuda.stream(sa):
        got_long = K().dense_attention(qb, kb, vb)
    with torch.cuda.stream(sb):
        for o in got:
            short(o)
    torch.cuda.synchronize()
    assert torch.equal(got_long[0], want_long[0]) and torch.equal(got_long[1], want_long[1])
    for o in got:
        for a, b in zip(o, want):
            assert torch.equal(a, b)


def test_dense_attention_past_4_gib(dev):
    """q / k / v of 4.3 GB each (L = 75 600, H = 224: row offsets past 2^32 bytes; the kernels base a buffer
    resource at every token block, so no 32-bit offset spans the tensor): the last head's first and last (80-row)
    query tiles against float64."""
    Lb, Hb = 75600, 224
    log("dense attention past 4 GiB: L", Lb, "H", Hb)
    g = torch.Generator(device=dev).manual_seed(3)
    qb, kb, vb = (torch.randn(Lb, Hb, D, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
    assert qb.numel() * 2 > 2 ** 32
    out, lse = K().dense_attention(qb, kb, vb)
    torch.cuda.synchronize()
    h = Hb - 1
    kh, vh = kb[:, h].double().cpu(), vb[:, h].double().cpu()
    for r0, r1 in ((0, 128), (Lb - 80, Lb)):
        qh = qb[r0:r1, h].double().cpu()
        s = qh @ kh.T / math.sqrt(D)
        want_l = torch.logsumexp(s, -1)
        want_o = torch.softmax(s, -1) @ vh
        check_close(f"O rows {r0}..{r1}", f32(out[r0:r1, h]), want_o.numpy())
        check_close(f"LSE rows {r0}..{r1}", f32(lse[r0:r1, h]) / math.log2(math.e), want_l.numpy())
    del qb, kb, vb, out, lse
    torch.cuda.empty_cache()
