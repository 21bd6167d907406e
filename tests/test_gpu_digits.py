"""The grouped kernels' int8 digit images of the layer input, byte for byte
against the numpy restatement (tests/_digits.py) and within half a digit
step of x, from each of their three writers: the fused routing kernel
(rows staged in LDS, four threads per sub-group), the router of wide rows
and the image kernel of callers that route from their own logits (one
thread per sub-group).  Rows mix ordinary values with sub-groups that are
all zero, tiny (below the 1e-30 floor), very large, or one outlier among
small values."""
import numpy as np
import pytest

import llmpager_amd as lp
from _digits import assert_digit_images
from _gpu import DeviceLayer

pytestmark = pytest.mark.gpu


def _rows(T: int, H: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32)
    for t in range(T):
        g = lambda i: slice(32 * ((7 * t + i) % (H // 32)), 32 * ((7 * t + i) % (H // 32)) + 32)
        x[t, g(0)] = 0.0
        x[t, g(1)] *= np.float32(1e-33)
        x[t, g(2)] *= np.float32(3e29)
        x[t, g(3)] *= np.float32(1e-4)
        x[t, g(3).start + 5] = np.float32(250.0)
        x[t, g(4)] *= np.float32(1e-29)
    return x


def _images(cuda, L, x, how):
    T, H = x.shape
    lay = lp.ws_layout(L.desc, T)
    ws = cuda.alloc_device(lay.total)
    dx = cuda.upload(x)
    if how == "route":
        L.layer.route(dx, T, ws)
    else:
        # routing from given logits writes no images; the expert half writes them
        dlog = cuda.upload(np.zeros((T, L.E), np.float32))
        dh = cuda.upload(np.zeros((T, H), np.float32))
        L.layer.route_logits(dlog, T, ws)
        L.layer.experts(dx, dh, T, ws)
        cuda.free_device(dlog)
        cuda.free_device(dh)
    img = cuda.download(ws + lay.xd, (T, lp.dimage_bytes(H)), np.uint8)
    cuda.free_device(ws)
    cuda.free_device(dx)
    return img


@pytest.mark.parametrize("T,how", [(1, "route"), (8, "route"), (20, "route"), (8, "experts"), (70, "route")])
def test_digit_images_config1(cuda, T, how):
    L = DeviceLayer(cuda, H=2048, I=768, E=128, k=8, group=32, seed=3)
    x = _rows(T, 2048, 10 + T)
    assert_digit_images(_images(cuda, L, x, how), x)
    L.free()


def test_digit_images_ragged_width(cuda):
    # 1408 columns: 44 sub-groups, padded to 44 (a multiple of 4); a width
    # whose rows the fused kernel cannot stage (config 4's 4096) goes through
    # the router of wide rows
    for H, I in ((1408, 256), (4096, 512)):
        L = DeviceLayer(cuda, H=H, I=I, E=16, k=4, group=32, seed=4)
        x = _rows(5, H, H)
        assert_digit_images(_images(cuda, L, x, "route"), x)
        L.free()
