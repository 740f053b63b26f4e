"""GPU backends: the kernel set is chosen from the device that holds q / k / v (reference echosparse/backends.py).

    gpu="auto"      gfx950 (MI355X) -> "mi355x"
    gpu="mi355x"    HIP kernels of `kernels.gfx950`; needs a gfx950 device

The reference resolves NVIDIA compute capabilities (h100 / b200 / rtx5090); this build resolves the AMD
architecture name (torch.cuda.get_device_properties(device).gcnArchName). The choice is made at the first
attention call, so a pipeline built on the CPU resolves it on the device it actually runs on.
"""
import importlib

import torch

GPUS = {"mi355x": "gfx950"}          # name -> AMD architecture
_NAMES = {arch: name for name, arch in GPUS.items()}


def check_name(gpu):
    if gpu not in ("auto", *GPUS):
        raise ValueError(f"gpu must be 'auto' or 'mi355x', not {gpu!r}")


def device_arch(device):
    """AMD architecture of a device, e.g. 'gfx950' (feature suffixes such as ':sramecc+' dropped)."""
    return torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]


def resolve(gpu, device):
    """Backend name for `gpu` ("auto" or "mi355x") on `device`; raises if they do not match."""
    check_name(gpu)
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError(f"EchoSparse runs on GPU tensors; got a tensor on {device}")
    arch = device_arch(device)
    found = _NAMES.get(arch)
    if gpu == "auto":
        if found is None:
            raise RuntimeError(f"{device} is {arch}; EchoSparse on ROCm supports gfx950 (MI355X) GPUs")
        return found
    if found != gpu:
        hint = f"use gpu='auto' or gpu='{found}'" if found else "no EchoSparse backend supports this GPU"
        raise RuntimeError(f"gpu='{gpu}' needs architecture {GPUS[gpu]}, but {device} is {arch}; {hint}")
    return gpu


def kernels(name):
    """Kernel module of a backend (imported on first use)."""
    return importlib.import_module(f"self_trainable_or_free_attn_amd.kernels.{GPUS[name]}")
