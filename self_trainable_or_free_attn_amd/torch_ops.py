"""Torch operator registration of the C ABI: every stream-taking entry point of include/echosparse_hip.h and
include/vsa_hip.h becomes the operator torch.ops.echosparse_gfx950.<entry point>, with the header's argument names
and order (the stream is torch's current HIP stream of the tensors' device).

The C++ registration (csrc/torch/ops.cpp) is generated from the headers, so the operator set can not drift from
the ABI:
  * a pointer parameter becomes an optional Tensor (None = NULL); a non-const pointer is declared mutable
    (Tensor(a!)?), so functionalisation and torch.compile see which arguments an operator writes
  * int / unsigned / size_t / long long become int, float / double become float; an int that does not fit the C
    type is refused (no silent wrap)
  * every tensor must be contiguous (a strided view would hand the kernel the wrong rows) and of the dtype its C
    type names: float* float32, int* / unsigned* int32 (or uint32), uint8_t* uint8 (or bool), const void* bf16
    or float16 (the token tensors), void* also float32 (outputs some entry points write in fp32 on request), and
    a void* named workspace any dtype
  * every operator returns nothing, like the C functions; a failing status raises RuntimeError with
    es_last_error_string(), a host tensor is refused before any launch
  * implementations for the CUDA (HIP) dispatch key, CPU (which only refuses host tensors) and Meta (no work, for
    fake-tensor tracing)
The reference registers its native op set as a pybind11 module (csrc/vsa/vsa2_api.cpp:904-941); here the same role
is played by torch.library (TORCH_LIBRARY), loaded with torch.ops.load_library.

The library is built by build_lib.build() (g++, host code only) into lib/libechosparse_torch.so. It does not link
libechosparse_hip.so: its C symbols resolve against the copy the ctypes binding loaded with RTLD_GLOBAL, so an
alternative build of the ABI (ECHOSPARSE_HIP_LIB) serves both bindings.
"""
import os
import re
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HEADERS = [os.path.join(ROOT, "include", h) for h in ("echosparse_hip.h", "vsa_hip.h")]
SOURCE = os.path.join(HERE, "csrc", "torch", "ops.cpp")
LIB = os.path.join(HERE, "lib", "libechosparse_torch.so")
NAMESPACE = "echosparse_gfx950"

_INT = {"int", "unsigned", "unsigned int", "size_t", "long long", "long"}
_FLOAT = {"float", "double"}


def _strip_comments(text):
    return re.sub(r"/\*.*?\*/", " ", re.sub(r"//[^\n]*", " ", text), flags=re.S)


def entry_points():
    """[(name, [(c_type, arg_name), ...])] of every declaration `int name(..., hipStream_t stream);`."""
    out = []
    for path in HEADERS:
        text = _strip_comments(open(path).read())
        for name, args in re.findall(r"\bint\s+((?:es|vsa)_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
            params = []
            for a in args.split(","):
                a = " ".join(a.split())
                m = re.match(r"(.*?)([A-Za-z_][A-Za-z0-9_]*)$", a)
                ctype, pname = m.group(1).strip(), m.group(2)
                params.append((ctype, pname))
            if not params or params[-1][0] != "hipStream_t":
                continue
            out.append((name, params[:-1]))
    return out


def _kind(ctype):
    if "*" in ctype:
        return "ptr_out" if not ctype.startswith("const") else "ptr_in"
    if ctype in _INT:
        return "int"
    if ctype in _FLOAT:
        return "float"
    raise ValueError(f"unsupported C parameter type {ctype!r}")


def _dtype_kind(ctype, pname):
    """The dtype check of a pointer parameter: ES_F32, ES_I32, ES_U8, ES_HALF, ES_OUT or ES_ANY."""
    base = ctype.replace("const", "").replace("*", "").strip()
    if base == "void":
        if pname == "workspace":
            return "ES_ANY"
        # a written token tensor may be an fp32 output (out_fp32 / accumulate variants)
        return "ES_HALF" if ctype.startswith("const") else "ES_OUT"
    return {"float": "ES_F32", "int": "ES_I32", "unsigned": "ES_I32", "uint8_t": "ES_U8"}[base]


_INT_RANGE = {"int": "ES_INT", "unsigned": "ES_UINT", "unsigned int": "ES_UINT", "size_t": "ES_SIZE",
              "long long": "ES_LL", "long": "ES_LL"}


def _schema(name, params):
    parts, alias = [], 0
    for ctype, pname in params:
        k = _kind(ctype)
        if k == "ptr_in":
            parts.append(f"Tensor? {pname}")
        elif k == "ptr_out":
            tag = "abcdefghijklmnopqrstuvwxyz"[alias]
            alias += 1
            parts.append(f"Tensor({tag}!)? {pname}")
        else:
            parts.append(f"{k} {pname}")
    return f"{name}({', '.join(parts)}) -> ()"


def _cxx_params(params):
    out = []
    for ctype, pname in params:
        k = _kind(ctype)
        if k.startswith("ptr"):
            out.append(f"const c10::optional<at::Tensor>& {pname}")
        elif k == "int":
            out.append(f"int64_t {pname}")
        else:
            out.append(f"double {pname}")
    return ", ".join(out)


def source():
    """The generated C++ registration."""
    eps = entry_points()
    lines = [
        "// Generated by self_trainable_or_free_attn_amd/torch_ops.py from include/echosparse_hip.h and",
        "// include/vsa_hip.h: one torch operator per stream-taking C entry point. Do not edit by hand.",
        '#include "../../../include/vsa_hip.h"',
        "",
        "#include <ATen/core/Tensor.h>",
        "#include <c10/core/DeviceGuard.h>",
        "#include <c10/hip/HIPStream.h>",
        "#include <torch/library.h>",
        "",
        "#include <cstdint>",
        "#include <initializer_list>",
        "",
        "namespace {",
        "",
        "// the device, guard and current stream of a call; refuses host tensors and tensors on two devices",
        "struct Call {",
        "  const char* name;",
        "  c10::optional<c10::Device> dev;",
        "  Call(const char* n, std::initializer_list<const c10::optional<at::Tensor>*> ts) : name(n) {",
        "    for (const auto* t : ts) {",
        "      if (!t->has_value()) continue;",
        "      const at::Tensor& x = **t;",
        "      TORCH_CHECK(x.is_cuda(), name, \": every tensor argument must live on the GPU (got a \", x.device(),",
        "                  \" tensor)\");",
        "      if (!dev) dev = x.device();",
        "      TORCH_CHECK(x.device() == *dev, name, \": tensors on two devices (\", *dev, \" and \", x.device(), \")\");",
        "    }",
        "  }",
        "};",
        "",
        "enum EsDtype { ES_F32, ES_I32, ES_U8, ES_HALF, ES_OUT, ES_ANY };",
        "",
        "// the pointer of an optional tensor argument after checking its layout and its dtype against the C type",
        "inline void* es_op_data(const char* name, const char* arg, const c10::optional<at::Tensor>& t, EsDtype kind) {",
        "  if (!t.has_value()) return nullptr;",
        "  const at::Tensor& x = *t;",
        "  TORCH_CHECK(x.is_contiguous(), name, \": argument \", arg, \" must be contiguous\");",
        "  const at::ScalarType s = x.scalar_type();",
        "  bool ok = true;",
        "  const char* want = \"\";",
        "  switch (kind) {",
        "    case ES_F32: ok = s == at::kFloat; want = \"float32\"; break;",
        "    case ES_I32: ok = s == at::kInt || s == at::kUInt32; want = \"int32\"; break;",
        "    case ES_U8: ok = s == at::kByte || s == at::kBool; want = \"uint8\"; break;",
        "    case ES_HALF: ok = s == at::kBFloat16 || s == at::kHalf; want = \"bfloat16 or float16\"; break;",
        "    case ES_OUT:",
        "      ok = s == at::kBFloat16 || s == at::kHalf || s == at::kFloat;",
        "      want = \"bfloat16, float16 or float32\";",
        "      break;",
        "    case ES_ANY: break;",
        "  }",
        "  TORCH_CHECK(ok, name, \": argument \", arg, \" must be \", want, \" (got \", s, \")\");",
        "  return x.data_ptr();",
        "}",
        "",
        "enum EsInt { ES_INT, ES_UINT, ES_SIZE, ES_LL };",
        "",
        "// an integer argument, refused if it does not fit the C parameter type",
        "inline int64_t es_op_int(const char* name, const char* arg, int64_t v, EsInt kind) {",
        "  const bool ok = kind == ES_INT    ? v >= INT32_MIN && v <= INT32_MAX",
        "                : kind == ES_UINT   ? v >= 0 && v <= int64_t(UINT32_MAX)",
        "                : kind == ES_SIZE   ? v >= 0",
        "                                    : true;",
        "  TORCH_CHECK(ok, name, \": argument \", arg, \" = \", v, \" is out of range for its C type\");",
        "  return v;",
        "}",
        "",
        "inline void es_op_check(const char* name, int status) {",
        "  TORCH_CHECK(status == 0, name, \" failed (status \", status, \"): \", es_last_error_string());",
        "}",
        "",
        "}  // namespace",
        "",
    ]
    for name, params in eps:
        tensors = [p for c, p in params if "*" in c]
        args = []
        for ctype, pname in params:
            k = _kind(ctype)
            if k.startswith("ptr"):
                args.append(f"static_cast<{ctype}>(es_op_data(\"{name}\", \"{pname}\", {pname}, "
                            f"{_dtype_kind(ctype, pname)}))")
            elif k == "int":
                args.append(f"static_cast<{ctype}>(es_op_int(\"{name}\", \"{pname}\", {pname}, "
                            f"{_INT_RANGE[ctype]}))")
            else:
                args.append(f"static_cast<{ctype}>({pname})")
        lines += [
            f"static void op_{name}({_cxx_params(params)}) {{",
            f"  const Call es_op_call(\"{name}\", {{{', '.join('&' + t for t in tensors)}}});",
            "  c10::OptionalDeviceGuard es_op_guard(es_op_call.dev);",
            "  const hipStream_t es_op_stream =",
            "      es_op_call.dev ? c10::hip::getCurrentHIPStream(es_op_call.dev->index()).stream() : nullptr;",
            f"  es_op_check(\"{name}\", {name}({', '.join(args + ['es_op_stream'])}));",
            "}",
            f"static void meta_{name}({_cxx_params(params)}) {{}}",
            "",
        ]
    lines.append(f"TORCH_LIBRARY({NAMESPACE}, m) {{")
    for name, params in eps:
        lines.append(f"  m.def(\"{_schema(name, params)}\");")
    lines.append("}")
    for key in ("CUDA", "CPU", "Meta"):
        lines.append(f"TORCH_LIBRARY_IMPL({NAMESPACE}, {key}, m) {{")
        for name, _ in eps:
            fn = f"meta_{name}" if key == "Meta" else f"op_{name}"
            lines.append(f"  m.impl(\"{name}\", TORCH_FN({fn}));")
        lines.append("}")
    return "\n".join(lines) + "\n"


def generate():
    """Write csrc/torch/ops.cpp if the headers changed it; returns its path."""
    text = source()
    os.makedirs(os.path.dirname(SOURCE), exist_ok=True)
    if not os.path.exists(SOURCE) or open(SOURCE).read() != text:
        with open(SOURCE, "w") as f:
            f.write(text)
    return SOURCE


def build(verbose=False):
    """Generate and compile lib/libechosparse_torch.so (host C++ against the installed torch)."""
    import torch.utils.cpp_extension as ce
    src = generate()
    tlib = os.path.join(os.path.dirname(ce.__file__), "..", "lib")
    incs = [f"-I{p}" for p in ce.include_paths(device_type="cuda")]
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM", *incs, src,
           "-o", LIB + ".tmp", f"-L{os.path.abspath(tlib)}", "-lc10", "-lc10_hip", "-ltorch_cpu"]
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"torch operator library failed to build:\n{r.stderr[-4000:]}")
    os.replace(LIB + ".tmp", LIB)
    if verbose:
        print(f"built {LIB} ({len(entry_points())} operators)")
    return LIB
