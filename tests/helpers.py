"""Shared test helpers: seeded inputs (generated on the CPU, then copied to the GPU so the oracle sees the same
values) and the tolerance checks of the hot path (max-abs 2e-2 and relative L2 1e-2 for floating-point outputs)."""
import numpy as np
import torch

MAX_ABS = 2e-2
REL_L2 = 1e-2


def structured_qkv(L, H, D=128, seed=0, steps=1, noise=0.05):
    """Inputs of `steps` consecutive denoising steps with local structure: a fixed smooth base per tensor (sines of
    position with random per-channel frequency and phase, amplitude 3) plus small per-step noise; bf16, (L, H, D)
    on the CPU. The same construction idea as the reference's test inputs (tests/test_attention.py:17-30)."""
    g = torch.Generator().manual_seed(seed)
    pos = torch.arange(L, dtype=torch.float32)[:, None, None] / 300.0
    freq = torch.randn(1, H, D, generator=g)
    base = [torch.sin(pos * freq + torch.randn(1, H, D, generator=g)) * 3.0 for _ in range(3)]
    out = []
    for _ in range(steps):
        out.append([(b + noise * torch.randn(b.shape, generator=g)).to(torch.bfloat16) for b in base])
    return out


def f32(x):
    """torch tensor (any dtype, any device) -> numpy float32."""
    return x.detach().float().cpu().numpy()


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def check_close(name, got, ref, max_abs=MAX_ABS, rel=REL_L2, mask=None):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    if mask is not None:
        got, ref = got[mask], ref[mask]
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    err = float(np.abs(got - ref).max()) if got.size else 0.0
    r = rel_l2(got, ref)
    assert err <= max_abs and r <= rel, f"{name}: max-abs {err:.3g} (<= {max_abs}), rel-L2 {r:.3g} (<= {rel})"
    return err, r


def bf16_max_abs(ref, floor=MAX_ABS):
    """The max-abs bound for a bf16-stored output: 2e-2, or half a bf16 step at the largest magnitude when that is
    larger (a bf16 value of |x| in [2^e, 2^(e+1)) is only defined to 2^(e-8)), so gradients of magnitude > 4 are
    held to their storage precision while the rel-L2 bound stays 1e-2."""
    return max(floor, 2.0 ** -8 * float(np.abs(np.asarray(ref, np.float64)).max(initial=0.0)))
