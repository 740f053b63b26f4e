"""es_representatives_noalloc (the allocation-free twin of es_representatives, workspace in a device array inside
the library) against es_representatives with a caller workspace, through the C ABI: two calls in a row, the second
with a smaller input (it must not depend on what the first left in the shared array), outputs bytes-identical
(same kernels, same arithmetic); and the size limit refused with a clear error."""
import math

import pytest
import torch

from helpers import structured_qkv

pytestmark = pytest.mark.gpu


def _lib():
    from self_trainable_or_free_attn_amd import _lib
    return _lib


def _outputs(L, H, dev):
    nb = -(-L // 64)
    nb4 = (nb + 1) * 4
    return dict(k=torch.zeros(H, nb4, 128, device=dev, dtype=torch.bfloat16),
                v=torch.zeros(H, nb4, 128, device=dev, dtype=torch.bfloat16),
                lc=torch.full((H, nb4), -math.inf, device=dev),
                km=torch.full((nb, H, 128), 3.0, device=dev, dtype=torch.bfloat16),
                vm=torch.full((nb, H, 128), 3.0, device=dev, dtype=torch.bfloat16))


def _with_workspace(q, k, v, o):
    L, H, D = q.shape
    ws = torch.empty(_lib().workspace_bytes(L, H, D), device=q.device, dtype=torch.uint8)
    _lib().call("es_representatives", q, k, v, o["k"], o["v"], o["lc"], o["km"], o["vm"], ws, ws.numel(), 6, L, H,
                D)


def _noalloc(q, k, v, o):
    L, H, D = q.shape
    _lib().call("es_representatives_noalloc", q, k, v, o["k"], o["v"], o["lc"], o["km"], o["vm"], 6, L, H, D)


def test_noalloc_representatives_match_workspace_entry_point(dev):
    got, want = [], []
    for L, H, seed in [(9000, 4, 21), (4200, 2, 22)]:
        print(f"[noalloc] L={L} H={H} seed={seed}", flush=True)
        (q, k, v), = structured_qkv(L, H, seed=seed)
        q, k, v = q.to(dev), k.to(dev), v.to(dev)
        o = _outputs(L, H, dev)
        _noalloc(q, k, v, o)
        got.append(o)
        w = _outputs(L, H, dev)
        _with_workspace(q, k, v, w)
        want.append(w)
    torch.cuda.synchronize()
    for o, w in zip(got, want):
        for name in o:
            assert torch.equal(o[name], w[name]), name
        assert torch.isfinite(o["lc"][:, :-4]).any()


def test_noalloc_representatives_refuses_sizes_beyond_its_scratch(dev):
    limit = int(_lib().lib().es_representatives_noalloc_limit())
    assert limit == 48 << 20
    L, H = 75600, 64
    assert _lib().workspace_bytes(L, H, 128) > limit
    assert _lib().workspace_bytes(75600, 40, 128) <= limit   # the Wan2.1-14B shape fits
    x = torch.zeros(64, 1, 128, device=dev, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="48 MiB device scratch"):
        _lib().call("es_representatives_noalloc", x, x, x, x, x, torch.zeros(4, device=dev), None, None, 6, L, H, 128)
