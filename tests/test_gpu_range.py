"""Activations with a wide dynamic range inside one 32-column sub-group.

The grouped decode kernels multiply digit images: per 32-column sub-group,
16-bit fixed point against the sub-group's own largest magnitude m (two int8
digits, sigma = m / 32639), so a sub-group that holds an outlier beside
N(0, 1) values keeps those small values only to within sigma / 2.  The
prefill GEMM reads fp16 images scaled per token row instead.  Residual
streams have such columns, so these tests put a few outliers of |x|
100..1000 into random sub-groups of every token, and scale whole token rows
by 30 and 1/30:

  - the device's digit images of x are byte-exact against the restatement
    of the per-sub-group rule (tests/_digits.py);
  - the layer delta matches the oracle fed with x as the digits carry it
    (x_rec, decoded from the device's images) to rel-L2 1e-4: what remains
    is the act rows' own digit rounding inside the down kernels and fp32
    accumulation order (a rule that quantised a row against its whole-row
    maximum, or lost an outlier, is far outside this);
  - the layer delta matches the oracle on the exact fp32 x to the north-star
    rel-L2 1e-3, decode (T = 1, 8, 32) and prefill (T = 256, the grouped
    GEMMs), every token checked."""
import numpy as np
import pytest

import llmpager_amd as lp
import _oracle as O
from _digits import assert_digit_images, decode_image
from _gpu import DeviceLayer, rel_l2

pytestmark = pytest.mark.gpu

H, I, E, K = 2048, 768, 128, 8


def wide_rows(T: int, seed: int) -> np.ndarray:
    """N(0, 1) rows, three sub-groups per token carrying one outlier of
    magnitude 100..1000 each; rows 1 and 2 (when present) scaled by 30 and
    1/30."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32)
    for t in range(T):
        for g in rng.choice(H // 32, 3, replace=False):
            c = 32 * g + rng.integers(32)
            x[t, c] = np.float32(rng.choice([-1.0, 1.0]) * rng.uniform(100.0, 1000.0))
    if T > 1:
        x[1] *= np.float32(30.0)
    if T > 2:
        x[2] *= np.float32(1.0 / 30.0)
    return x


@pytest.fixture(scope="module")
def layer(cuda):
    L = DeviceLayer(cuda, H=H, I=I, E=E, k=K, group=32, seed=61)
    yield L
    L.free()


def _run(cuda, L, x, h):
    T = x.shape[0]
    lay = lp.ws_layout(L.desc, T)
    ws = cuda.alloc_device(lay.total)
    dx, dh = cuda.upload(x), cuda.upload(h)
    L.layer.forward(dx, dh, T, ws)
    got = cuda.download(dh, (T, H), np.float32)
    glog = cuda.download(ws + lay.logits, (T, E), np.float32)
    xd = cuda.download(ws + lay.xd, (T, lp.dimage_bytes(H)), np.uint8)
    status = L.layer.status(ws, T)
    for p in (ws, dx, dh):
        cuda.free_device(p)
    assert status[1] == 0
    return got, glog, xd, lay


@pytest.mark.parametrize("T", [1, 8, 32])
def test_decode_wide_range_subgroups(cuda, layer, T):
    x = wide_rows(T, 700 + T)
    h = np.random.default_rng(800 + T).standard_normal((T, H)).astype(np.float32)
    got, glog, xd, _ = _run(cuda, layer, x, h)
    assert_digit_images(xd, x)
    # the oracle on x as the digits carry it, routed by the device's logits
    x_rec = np.stack([decode_image(xd[t], H)[0] for t in range(T)]).astype(np.float32)
    small = np.abs(x) < 5
    assert np.abs(x_rec - x)[small].max() > 1e-3   # the outliers' sub-groups did lose precision
    want_rec = O.moe_layer(layer.oracle_desc(), layer.oracle_blobs(), x_rec, h.copy(), logits_in=glog, threads=8)[0]
    err_rec = rel_l2(got - h, want_rec - h)
    assert err_rec <= 1e-4, err_rec
    # the contract: the oracle on the exact x
    want = O.moe_layer(layer.oracle_desc(), layer.oracle_blobs(), x, h.copy(), logits_in=glog, threads=8)[0]
    err = rel_l2(got - h, want - h)
    assert err <= 1e-3, err


def test_prefill_wide_range_subgroups(cuda, layer):
    T = 256
    x = wide_rows(T, 900)
    h = np.random.default_rng(901).standard_normal((T, H)).astype(np.float32)
    got, glog, _, lay = _run(cuda, layer, x, h)
    assert lay.tiles != lay.actimg, "this shape must take the GEMM path"
    want = O.moe_layer(layer.oracle_desc(), layer.oracle_blobs(), x, h.copy(), logits_in=glog, threads=8)[0]
    err = rel_l2(got - h, want - h)
    assert err <= 1e-3, err
