"""Build libechosparse_hip.so in-tree with hipcc for gfx950 (python -m self_trainable_or_free_attn_amd.build_lib), then
the torch operator library over it (torch_ops.py, lib/libechosparse_torch.so).

Every HIP source under csrc/ is compiled to an object in parallel and linked into lib/libechosparse_hip.so; the
VSA sources (vsa_*.hip) are compiled a second time with -DES_ELEM_F16 for their fp16 entry points (suffix _f16).
Flags: -O3, gfx950 only, and packed FP32 instructions disabled (-Xclang -target-feature -Xclang -packed-fp32-ops).
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libechosparse_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-Wno-unused-result"] + os.environ.get("ECHOSPARSE_HIP_CFLAGS", "").split()


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def units():
    """(source, extra flags, object suffix) for every compilation: each source once, the VSA ones also for fp16."""
    out = []
    for src in sources():
        out.append((src, [], ""))
        if os.path.basename(src).startswith("vsa_"):
            out.append((src, ["-DES_ELEM_F16"], ".f16"))
    return out


def _compile(unit, obj_dir):
    src, extra, suffix = unit
    obj = os.path.join(obj_dir, os.path.basename(src) + suffix + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC, *FLAGS, *extra, *lang, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj


def build(verbose=False, out=None):
    """Compile every source and link the shared library (to `out`, default lib/libechosparse_hip.so); returns its
    path."""
    lib_path = out or LIB
    obj_dir = os.path.join(HERE, "_build", os.path.basename(lib_path))
    os.makedirs(obj_dir, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = units()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda u: _compile(u, obj_dir), srcs))
    os.makedirs(os.path.dirname(lib_path), exist_ok=True)
    tmp = lib_path + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, lib_path)
    if verbose:
        print(f"built {lib_path} from {len(srcs)} compilations")
    if out is None:  # the torch operators over the default build
        from . import torch_ops
        torch_ops.build(verbose=verbose)
    return lib_path


if __name__ == "__main__":
    build(verbose=True, out=sys.argv[1] if len(sys.argv) > 1 else None)
    sys.exit(0)
