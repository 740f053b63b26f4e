"""Seeded synthetic inputs for the benchmark configurations (no network, no checkpoints).

`fourier_qkv` builds the EchoSparse headline inputs: tokens on a (frames, height, width) latent grid stored in
Morton order (the order the reference's Wan integration uses, echosparse/models/common.py:39-53), Q and K from one
low-frequency random Fourier field of grid position (8 modes per axis, amplitude ~1/mode) plus 0.3 N(0, 1) noise
each, V ~ N(0, 1). Each head's Q / K scale is chosen by bisection so the mean entropy of a row's softmax over all
keys is `entropy_frac` * ln(L).
"""
import math

import torch


def morton_order(t, y, x):
    """Permutation sorting (t, y, x) coordinates along a 3D Morton curve (bit i of x, y, t at 3i, 3i+1, 3i+2),
    and its inverse."""
    code = torch.zeros_like(x)
    for bit in range(21):
        code |= ((x >> bit) & 1) << (3 * bit)
        code |= ((y >> bit) & 1) << (3 * bit + 1)
        code |= ((t >> bit) & 1) << (3 * bit + 2)
    perm = torch.argsort(code)
    return perm, torch.argsort(perm)


def grid_morton_order(frames, height, width, device="cpu"):
    t, y, x = torch.meshgrid(torch.arange(frames), torch.arange(height), torch.arange(width), indexing="ij")
    perm, inv = morton_order(t.flatten(), y.flatten(), x.flatten())
    return perm.to(device), inv.to(device)


def _field_features(grid, modes, device):
    """(L, 6 * modes) cos / sin features of the grid positions in raster order, amplitude 1 / mode."""
    F, Y, X = grid
    t, y, x = torch.meshgrid(torch.arange(F, device=device), torch.arange(Y, device=device),
                             torch.arange(X, device=device), indexing="ij")
    feats = []
    for coord, n in ((t, F), (y, Y), (x, X)):
        c = coord.flatten().float() / n
        for m in range(1, modes + 1):
            ang = 2 * math.pi * m * c / 2      # half-period base: the lowest mode varies once over the axis
            feats += [torch.cos(ang) / m, torch.sin(ang) / m]
    return torch.stack(feats, 1)


def _mean_entropy(q, k, rows, D):
    """Mean natural entropy of softmax(q_r . k / sqrt(D)) over all keys for the sampled rows. q, k: (L, D)."""
    s = (q[rows].float() @ k.float().T) / math.sqrt(D)
    p = torch.softmax(s, -1)
    return float(-(p * torch.log(p.clamp_min(1e-30))).sum(-1).mean())


def fourier_qkv(grid=(21, 45, 80), H=40, D=128, seed=2, modes=8, noise=0.3, entropy_frac=0.2, device="cuda",
                dtype=torch.bfloat16, sample_rows=256, pad_to=None):
    """Returns q, k, v as (L, H, D) tensors in Morton token order (L = frames * height * width) and the per-head
    scales. `pad_to`: optional padded length; extra rows are zero (the kernels only read rows < L)."""
    g = torch.Generator(device=device).manual_seed(seed)
    L = grid[0] * grid[1] * grid[2]
    feats = _field_features(grid, modes, device)                      # (L, 6m), raster order
    perm, _ = grid_morton_order(*grid, device=device)
    feats = feats[perm]
    nf = feats.shape[1]
    rows = torch.randint(0, L, (sample_rows,), device=device, generator=g)
    target = entropy_frac * math.log(L)
    q = torch.empty(L, H, D, device=device, dtype=dtype)
    k = torch.empty_like(q)
    scales = []
    for h in range(H):
        W = torch.randn(nf, D, device=device, generator=g)
        field = feats @ W
        field = field / field.std()
        qh = field + noise * torch.randn(L, D, device=device, generator=g)
        kh = field + noise * torch.randn(L, D, device=device, generator=g)
        lo, hi = math.log(0.05), math.log(20.0)        # bisection on log(scale): entropy falls as scale grows
        for _ in range(24):
            mid = 0.5 * (lo + hi)
            s = math.exp(mid)
            e = _mean_entropy(qh * s, kh * s, rows, D)
            if e > target:
                lo = mid
            else:
                hi = mid
        s = math.exp(0.5 * (lo + hi))
        scales.append(s)
        q[:, h] = (qh * s).to(dtype)
        k[:, h] = (kh * s).to(dtype)
    v = torch.randn(L, H, D, device=device, generator=g).to(dtype)
    if pad_to is not None and pad_to > L:
        pad = lambda x: torch.cat([x, torch.zeros(pad_to - L, H, D, device=device, dtype=dtype)])
        q, k, v = pad(q), pad(k), pad(v)
    return q, k, v, scales


def perturbed(x, frac=0.01, seed=0):
    """x + frac * std(x) * N(0, 1), in x's dtype (the 'previous step' inputs)."""
    g = torch.Generator(device=x.device).manual_seed(seed)
    n = torch.randn(x.shape, device=x.device, generator=g)
    return (x.float() + frac * x.float().std() * n).to(x.dtype)
