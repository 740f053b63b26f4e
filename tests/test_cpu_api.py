"""Host logic and the C ABI without a GPU: backend resolution, the per-layer state sizes the reference pins, and that
libechosparse_hip.so loads and exports every entry point include/echosparse_hip.h declares (no compute calls)."""
import ctypes
import os
import re
import subprocess
import sys
import types

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture
def arch(monkeypatch):
    def set_arch(name):
        props = types.SimpleNamespace(gcnArchName=name)
        monkeypatch.setattr(torch.cuda, "get_device_properties", lambda device=None: props)
    return set_arch


def test_auto_follows_the_device(arch):
    from self_trainable_or_free_attn_amd import backends
    arch("gfx950:sramecc+:xnack-")
    assert backends.resolve("auto", "cuda:0") == "mi355x"
    assert backends.resolve("mi355x", torch.device("cuda", 0)) == "mi355x"


def test_mismatch_and_unsupported_devices_fail(arch):
    from self_trainable_or_free_attn_amd import backends
    arch("gfx942")
    with pytest.raises(RuntimeError, match="gpu='mi355x' needs architecture gfx950, but cuda:0 is gfx942"):
        backends.resolve("mi355x", "cuda:0")
    with pytest.raises(RuntimeError, match="is gfx942; EchoSparse on ROCm supports gfx950"):
        backends.resolve("auto", "cuda:0")
    with pytest.raises(ValueError, match="GPU tensors"):
        backends.resolve("auto", "cpu")
    with pytest.raises(ValueError, match="gpu must be"):
        backends.resolve("h100", "cuda:0")


def test_attention_resolves_at_the_first_call():
    from self_trainable_or_free_attn_amd import EchoSparseAttention
    attn = EchoSparseAttention(gpu="mi355x")
    assert attn.backend is None
    q = torch.zeros(1, 128, 1, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensors"):
        attn(q, q, q, step=0, branch=0, layer=0)
    with pytest.raises(ValueError, match="gpu must be"):
        EchoSparseAttention(gpu="5090")
    with pytest.raises(AssertionError):
        EchoSparseAttention(dense_steps=1)


def test_import_does_not_load_kernels():
    code = ("import sys; sys.path.insert(0, %r); import self_trainable_or_free_attn_amd; "
            "print(any(m.endswith('kernels.gfx950') or m.endswith('._lib') for m in sys.modules))" % ROOT)
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, check=True).stdout
    assert out == "False\n"


@pytest.mark.parametrize("L, H, layers, branches, expected", [
    (75600, 40, 39, 2, 1888174080),      # Wan2.1-14B 720p, layers 1-39, CFG
    (118839, 24, 60, 1, 1369866240),     # HunyuanVideo 720p: 118800 video + 39 text tokens
    (38247, 56, 49, 1, 630110208),       # MiniMax-H3 768p, layers 1-49
])
def test_state_size(L, H, layers, branches, expected):
    """Persistent per-layer state (offsets of every branch + bit plans) equals the reference's pinned byte counts
    (reference tests/test_api.py:129-143)."""
    from self_trainable_or_free_attn_amd.attention import _CompactState
    st = _CompactState(L, H, "meta")
    for branch in range(branches):
        st.offset(branch)
    for plan in range(branches):
        st.plan(plan)
    tensors = [*st.offsets.values(), *(t for p in st.plans for t in p)]
    assert layers * sum(t.numel() * t.element_size() for t in tensors) == expected


def test_budget_matches_reference_rule():
    from self_trainable_or_free_attn_amd import EchoSparseAttention
    attn = EchoSparseAttention(density=0.1)
    assert attn._budget(1182) == (118, 355) and attn._budget(65) == (6, 20)
    assert EchoSparseAttention(density=1.0)._budget(65) == (65, 0)


HEADERS = ("echosparse_hip.h", "vsa_hip.h")


def header_text():
    text = "".join(open(os.path.join(ROOT, "include", h)).read() for h in HEADERS)
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def declared_entry_points():
    return sorted(set(re.findall(r"\b((?:es|vsa)_[a-z0-9_]+)\s*\(", header_text())))


def library():
    from self_trainable_or_free_attn_amd import _lib, build_lib
    if not os.path.exists(_lib.LIB_PATH):
        build_lib.build()
    return ctypes.CDLL(_lib.LIB_PATH)


def test_library_exports_every_declared_entry_point():
    names = declared_entry_points()
    assert len(names) >= 35 and "es_sparse_attention" in names and "vsa_attn_bwd_kv" in names
    so = library()
    missing = [n for n in names if not hasattr(so, n)]
    assert not missing, missing
    so.es_abi_version.restype = ctypes.c_int
    assert so.es_abi_version() == 2


def test_ctypes_signatures_cover_the_header():
    """Every stream-taking entry point of the header has an argument list in the binding, with the header's
    argument count (the binding appends the stream)."""
    from self_trainable_or_free_attn_amd import _lib
    for name, args in re.findall(r"\b((?:es|vsa)_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", header_text()):
        n = len([a for a in args.split(",") if a.strip() and a.strip() != "void"])
        if "hipStream_t" in args:
            assert name in _lib.SIGNATURES, name
            assert len(_lib.SIGNATURES[name]) + 1 == n, name
        else:
            assert name in _lib.NO_STREAM, name


def test_argument_errors_are_reported_without_a_gpu():
    """Validation runs before any HIP call: a bad head dimension is reported with a message."""
    so = library()
    so.es_block_means.restype = ctypes.c_int
    so.es_last_error_string.restype = ctypes.c_char_p
    p = ctypes.c_void_p(16)
    st = so.es_block_means(p, p, p, p, ctypes.c_int(64), ctypes.c_int(1), ctypes.c_int(64), ctypes.c_void_p(0))
    assert st == 2 and b"head dimension must be 128" in so.es_last_error_string()
    st = so.es_block_means(None, p, p, p, ctypes.c_int(64), ctypes.c_int(1), ctypes.c_int(128), ctypes.c_void_p(0))
    assert st == 1 and b"null" in so.es_last_error_string()


def test_host_tensors_are_refused_before_any_launch():
    """A host tensor's address given to a kernel would fault the GPU: the binding refuses it first."""
    import torch
    from self_trainable_or_free_attn_amd import _lib
    x = torch.zeros(4)
    with pytest.raises(RuntimeError, match="must live on the GPU"):
        _lib.call("vsa_finalize", None, None, 0, x, x, 1, 64, 128)


def test_torch_operators_are_generated_from_the_header():
    """csrc/torch/ops.cpp is the generator's output for the current headers, and every stream-taking entry point is
    an operator with the header's argument names, non-const pointers declared as written (Tensor(x!)?)."""
    from self_trainable_or_free_attn_amd import _lib, torch_ops
    assert open(torch_ops.SOURCE).read() == torch_ops.source(), "run build_lib: ops.cpp is stale"
    if not os.path.exists(_lib.TORCH_LIB_PATH):
        from self_trainable_or_free_attn_amd import build_lib
        build_lib.build()
    ops = _lib.ops()
    eps = torch_ops.entry_points()
    assert {n for n, _ in eps} == set(_lib.SIGNATURES)
    for name, params in eps:
        schema = getattr(ops, name).default._schema
        assert [a.name for a in schema.arguments] == [p for _, p in params], name
        for a, (ctype, _) in zip(schema.arguments, params):
            written = a.alias_info is not None and a.alias_info.is_write
            assert written == ("*" in ctype and not ctype.startswith("const")), (name, a.name)
        assert len(schema.returns) == 0


def test_torch_operators_trace_with_meta_tensors_and_refuse_host_tensors():
    """Meta tensors run the no-op Meta kernel (fake-tensor tracing); host tensors are refused by name."""
    import torch
    from self_trainable_or_free_attn_amd import _lib
    ops = _lib.ops()
    m = torch.empty(64, 1, 128, dtype=torch.bfloat16, device="meta")
    mm = torch.empty(1, 1, 128, dtype=torch.bfloat16, device="meta")
    assert ops.es_block_means(m, m, mm, mm, 64, 1, 128) is None
    c = torch.zeros(64, 1, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="es_block_means: every tensor argument must live on the GPU"):
        ops.es_block_means(c, c, c[:1], c[:1], 64, 1, 128)


def test_block_count_limits_are_refused_before_any_launch():
    """Each VSA entry point with a block-count limit refuses a larger NB with a message, before any HIP call:
    route_rows, the three-tier kernels and the per-row tiers NB <= 8192, the global top-k and the CSR transpose
    NB <= 46 340; the limits themselves are accepted as far as that check."""
    so = library()
    so.es_last_error_string.restype = ctypes.c_char_p
    p = ctypes.c_void_p(256)
    i, ll, sz = ctypes.c_int, ctypes.c_longlong, ctypes.c_size_t
    null = ctypes.c_void_p(0)

    def route_rows(nb, bh_count=1):
        return so.vsa_route_rows(p, p, i(nb), i(64 * ((nb + 63) // 64)), i(0), i(bh_count), i(1), i(128), p, p, p, p,
                                 p, sz(1 << 40), null)

    def rep_fwd(nb):
        return so.vsa_rep_attn_fwd(p, p, p, p, p, p, i(0), p, p, p, p, p, p, p, p, p, p, i(1), i(nb * 64), i(128),
                                   i(4), i(8), null)

    def row_tiers(nb):
        return so.vsa_row_tiers(p, i(nb), i(0), i(1), i(0), i(nb + 1), p, p, p, p, p, p, null)

    def global_topk(nb):
        return so.vsa_global_topk(p, i(nb), i(0), i(1), ll(1), p, p, p, p, p, p, sz(0), null)

    def csr_transpose(nb):
        return so.vsa_csr_transpose(p, p, i(nb), i(0), i(1), p, p, p, sz(0), null)

    # (name, call, the largest NB, the refusal text). At the limit a later host check must fail instead, so that no
    # kernel ever sees these placeholder pointers: no (b, h) rows, phases 8, kab > NB, a workspace too small.
    cases = [("route_rows", route_rows, 8192, b"NB <= 8192"), ("rep_attn_fwd", rep_fwd, 8192, b"NB <= 8192"),
             ("row_tiers", row_tiers, 8192, b"NB <= 8192"), ("global_topk", global_topk, 46340, b"bad top-k shape"),
             ("csr_transpose", csr_transpose, 46340, b"NB <= 46340")]
    for name, call, limit, text in cases:
        assert call(limit + 1) != 0, name
        assert text in so.es_last_error_string(), (name, so.es_last_error_string())
        assert (call(limit, 0) if name == "route_rows" else call(limit)) != 0, name
        msg = so.es_last_error_string()
        assert text not in msg and msg, (name, msg)
