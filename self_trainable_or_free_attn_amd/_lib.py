"""Bindings of the C ABI in include/echosparse_hip.h and include/vsa_hip.h (libechosparse_hip.so, built in-tree by
build_lib).

Kernel calls (`call`) go through the torch operators torch.ops.echosparse_gfx950.<entry point> (torch_ops.py,
lib/libechosparse_torch.so): arguments are tensors (None = NULL) and Python scalars in the header's order, and each
call is enqueued on torch's current HIP stream of the tensors' device, so the kernels order with the surrounding
torch work exactly like the reference's launches do. The ctypes handle (`lib`) serves the entry points without a
stream (workspace sizes, limits, the error string) and tests that drive the C ABI directly.

There is no fallback: if either library is missing or fails to load, every kernel call raises.
"""
import ctypes
import numbers
import os

import torch

# ECHOSPARSE_HIP_LIB: load another build of the same ABI (development A/B measurements)
LIB_PATH = os.environ.get("ECHOSPARSE_HIP_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib",
                                                                "libechosparse_hip.so")
TORCH_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libechosparse_torch.so")

# the ES_ABI_VERSION of include/echosparse_hip.h these bindings follow; a library reporting another is refused
ABI_VERSION = 2

P, I, F, Z = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
LL, DB = ctypes.c_longlong, ctypes.c_double

# name -> argument types (the trailing hipStream_t is added below); mirrors include/echosparse_hip.h
SIGNATURES = {
    "es_block_attention": [P, P, P, P, P, P, I, P, P, P, P, F, I, I, I],
    "es_sparse_attention": [P, P, P, P, P, P, P, P, P, P, I, P, P, P, P, P, I, P, P, P, P, F, I, I, I, I],
    "es_exact_fallback": [P, P, P, P, P, P, I, P, P, I, I, I],
    "es_compensate_fallback": [P, P, P, P, P, P, P, I, I, I],
    "es_dense_attention": [P, P, P, P, P, I, I, I],
    "es_dense_attention_kv": [P, P, P, P, P, I, I, I, I],
    "es_block_means": [P, P, P, P, I, I, I],
    "es_estimate_skipped": [P, P, P, P, P, P, P, P, I, I, I],
    "es_full_step_scales": [P, P, P, P, I, I],
    "es_select_blocks": [P, P, P, P, P, P, P, P, P, I, P, I, I, I, I, I, I],
    "es_pack_plan": [P, P, I, I, I, I],
    "es_rebuild_plan": [P, P, I, P, P, P, P, P, I, P, P, I, I, I],
    "es_representatives": [P, P, P, P, P, P, P, P, P, Z, I, I, I, I],
    "es_representatives_noalloc": [P, P, P, P, P, P, P, P, I, I, I, I],
    # include/vsa_hip.h
    "vsa_pool": [P, P, P, P, P, P, P, P, P, P, I, I, I, I],
    "vsa_fuse_fwd": [P, P, P, P, P, I, I, I, I, I, I],
    "vsa_fuse_bwd": [P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I],
    "vsa_finalize": [P, P, I, P, P, I, I, I],
    "vsa_attn_fwd": [P, P, P, P, P, P, P, P, I, I, I],
    "vsa_attn_fwd_tasks": [P, P, P, P, P, P, P, I, P, P, P, P, I, I, I],
    "vsa_attn_bwd_kv": [P, P, P, P, P, P, P, P, P, P, P, I, P, P, I, I, I, I],
    "vsa_attn_bwd_kv_tasks": [P, P, P, P, P, P, P, P, P, P, I, P, P, I, P, P, P, P, I, I, I],
    "vsa_attn_bwd_q": [P, P, P, P, P, P, P, P, P, P, I, P, P, I, I, I],
    "vsa_attn_bwd_q_tasks": [P, P, P, P, P, P, P, P, P, P, I, P, I, P, P, I, I, I],
    "vsa_block_scores": [P, P, P, I, I, I, I, I],
    "vsa_route_rows": [P, P, I, I, I, I, I, I, P, P, P, P, P, Z],
    "vsa_row_topk": [P, I, I, I, I, P, P, P, P, P, Z],
    "vsa_router_lse": [P, P, P, P, I, I, I, I],
    "vsa_router_scores": [P, P, P, P, P, I, I, I, I, I, I],
    "vsa_global_topk": [P, I, I, I, LL, P, P, P, P, P, P, Z],
    "vsa_csr_transpose": [P, P, I, I, I, P, P, P, Z],
    "vsa_split_plan": [P, I, I, I, I, I, DB, DB, I, I, P, P, P],
    "vsa_split_merge_fwd": [P, P, P, P, I, P, P, P, I, I, I, I],
    "vsa_split_merge_sum": [P, P, P, I, P, I, P, P, P, I, I, I],
    "vsa_rep_build": [P, P, P, P, P, P, P, P, P, I, I, I, I],
    "vsa_rep_build_kmeans": [P, P, P, P, P, P, P, P, I, I, I, I, I, ctypes.c_uint],
    "vsa_row_tiers": [P, I, I, I, I, I, P, P, P, P, P, P],
    "vsa_rep_attn_fwd": [P, P, P, P, P, P, I, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I],
    "vsa_rep_attn_bwd_q": [P, P, P, P, P, P, I, P, P, P, P, P, P, P, P, P, P, P, P, I, P, P, I, I, I, I, I],
    "vsa_rep_bwd_tables": [P, P, P, P, P, I, P, P, P, P, P, P, I, I, I, I, I],
    "vsa_rep_unpool": [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I],
    "vsa_row_dot": [P, P, P, P, I, I, I],
    "vsa_tier_b_lists": [P, P, P, P, P, P, I, I],
}
# include/vsa_hip.h: the fp16 twins (suffix _f16) of the entry points that take token tensors, same arguments
F16_TWINS = ("vsa_pool", "vsa_fuse_fwd", "vsa_fuse_bwd", "vsa_finalize", "vsa_attn_fwd", "vsa_attn_fwd_tasks",
             "vsa_attn_bwd_kv", "vsa_attn_bwd_kv_tasks", "vsa_attn_bwd_q", "vsa_attn_bwd_q_tasks", "vsa_block_scores",
             "vsa_route_rows", "vsa_row_topk", "vsa_router_lse", "vsa_router_scores", "vsa_split_merge_fwd",
             "vsa_split_merge_sum", "vsa_rep_build", "vsa_rep_build_kmeans", "vsa_rep_attn_fwd", "vsa_rep_attn_bwd_q", "vsa_rep_bwd_tables",
             "vsa_rep_unpool", "vsa_row_dot")
SIGNATURES.update({n + "_f16": SIGNATURES[n] for n in F16_TWINS})
NO_STREAM = {"es_representatives_workspace": ([I, I, I], Z), "es_representatives_noalloc_limit": ([], Z), "es_last_error_string": ([], ctypes.c_char_p),
             "es_abi_version": ([], I), "vsa_topk_workspace": ([I, I], Z)}

_lib = None
_ops = None


def lib():
    """The loaded library (loaded on first use; raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m self_trainable_or_free_attn_amd.build_lib`")
        # RTLD_GLOBAL: the torch operator library resolves its C symbols against this copy
        so = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        for name, args in SIGNATURES.items():
            fn = getattr(so, name)
            fn.argtypes = [*args, P]
            fn.restype = I
        for name, (args, res) in NO_STREAM.items():
            fn = getattr(so, name)
            fn.argtypes = args
            fn.restype = res
        if so.es_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} implements ABI version {so.es_abi_version()}, these bindings follow "
                               f"version {ABI_VERSION}: rebuild it with build_lib")
        _lib = so
    return _lib


def ops():
    """torch.ops.echosparse_gfx950 (loaded on first use, after the C library; raises if it is not built)."""
    global _ops
    if _ops is None:
        lib()
        if not os.path.exists(TORCH_LIB_PATH):
            raise RuntimeError(f"{TORCH_LIB_PATH} is not built; run `python -m self_trainable_or_free_attn_amd.build_lib`")
        torch.ops.load_library(TORCH_LIB_PATH)
        _ops = torch.ops.echosparse_gfx950
    return _ops


def ptr(x):
    """Device pointer of a tensor (None -> NULL), for direct ctypes calls."""
    if x is None:
        return None
    return ctypes.c_void_p(x.data_ptr())


def call(name, *args):
    """Call an entry point through its torch operator on torch's current stream. A failing status raises
    RuntimeError with the library's message; a host tensor is refused before the launch (its address handed to a
    kernel would fault the GPU)."""
    getattr(ops(), name)(*map(_plain, args))


def _plain(a):
    """Tensors, None and Python scalars pass as they are; other numbers (numpy scalars) become int / float."""
    if a is None or isinstance(a, (torch.Tensor, bool, int, float)):
        return a
    return int(a) if isinstance(a, numbers.Integral) else float(a)


def workspace_bytes(L, H, D):
    return int(lib().es_representatives_workspace(L, H, D))


def topk_workspace_bytes(bh_count, NB):
    return int(lib().vsa_topk_workspace(bh_count, NB))
