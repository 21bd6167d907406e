"""The allocation-free layer entry point (lp_moe_forward_noalloc) against
lp_moe_forward with a caller workspace: the same kernels on the same inputs,
so the residual, the routing and the status words are identical.  Two calls
in a row share the built-in scratch; the second, smaller one must not see
the first one's tables."""
import numpy as np
import pytest

import llmpager_amd as lp
from _gpu import DeviceLayer

pytestmark = pytest.mark.gpu


def _fp32(n, seed):
    return np.random.default_rng(seed).standard_normal(n).astype(np.float32)


def _with_workspace(cuda, L, x, h):
    T = x.shape[0]
    lay = lp.ws_layout(L.desc, T)
    ws = cuda.alloc_device(lay.total)
    dx, dh = cuda.upload(x), cuda.upload(h)
    L.layer.forward(dx, dh, T, ws)
    out = cuda.download(dh, (T, L.H), np.float32)
    st = L.layer.status(ws, T)
    for p in (ws, dx, dh):
        cuda.free_device(p)
    return out, st


def test_noalloc_matches_forward(cuda):
    L = DeviceLayer(cuda, H=2048, I=768, E=128, k=8, group=32, seed=81)
    assert lp.lib().lp_noalloc_scratch_bytes() == 16 << 20
    for T, seed in ((32, 1), (8, 2)):   # the second call is smaller
        x = _fp32(T * 2048, 10 + seed).reshape(T, 2048)
        h = _fp32(T * 2048, 20 + seed).reshape(T, 2048)
        want, st = _with_workspace(cuda, L, x, h)
        assert st[1] == 0
        dx, dh = cuda.upload(x), cuda.upload(h)
        L.layer.forward_noalloc(dx, dh, T)
        got = cuda.download(dh, (T, 2048), np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), T
        for p in (dx, dh):
            cuda.free_device(p)
    # a batch whose workspace exceeds the scratch is refused before any launch
    T = 2048
    assert lp.ws_layout(L.desc, T).total > lp.lib().lp_noalloc_scratch_bytes()
    with pytest.raises(lp.LpError) as ei:
        L.layer.forward_noalloc(0, 0, T)
    assert ei.value.code == -2 and "scratch" in str(ei.value)
    L.free()
