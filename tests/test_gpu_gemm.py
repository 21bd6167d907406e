"""The prefill path: the grouped MFMA GEMMs (lp_gemm.hip) the experts phase
switches to once routed experts average 16+ tokens, against the oracle."""
import numpy as np
import pytest

import llmpager_amd as lp
import _oracle as O
from _gpu import DeviceLayer, rel_l2

pytestmark = pytest.mark.gpu


def _layer_vs_oracle(cuda, L: DeviceLayer, T: int, seed: int, logits=None, sample=None):
    H, E, k = L.H, L.E, L.k
    x = lp.synth_f32_bf16(T * H, 1.0, seed, 1).reshape(T, H)
    h = lp.synth_f32_bf16(T * H, 1.0, seed, 2).reshape(T, H)
    lay = lp.ws_layout(L.desc, T)
    assert lay.tiles != lay.actimg, "this shape must take the GEMM path"
    ws = cuda.alloc_device(lay.total)
    dx, dh = cuda.upload(x), cuda.upload(h)
    if logits is None:
        L.layer.forward(dx, dh, T, ws)
    else:
        dl = cuda.upload(np.ascontiguousarray(logits, np.float32))
        L.layer.route_logits(dl, T, ws)
        L.layer.experts(dx, dh, T, ws)
        cuda.free_device(dl)
    got = cuda.download(dh, (T, H), np.float32)
    status = L.layer.status(ws, T)
    got_logits = cuda.download(ws + lay.logits, (T, E), np.float32)
    for p in (ws, dx, dh):
        cuda.free_device(p)
    rows = np.arange(T) if sample is None else np.asarray(sample)
    want = O.moe_layer(L.oracle_desc(), L.oracle_blobs(), x[rows], h[rows].copy(),
                       logits_in=np.ascontiguousarray(got_logits[rows]), threads=8)[0]
    assert status[1] == 0
    err = rel_l2(got[rows] - h[rows], want - h[rows])
    assert err <= 1e-3, err
    return got_logits


def test_gemm_layer_small(cuda):
    # 128 tokens x top-4 over 16 experts: 32 pairs per expert on average
    L = DeviceLayer(cuda, H=512, I=256, E=16, k=4, group=32, seed=21, router_std=0.05)
    _layer_vs_oracle(cuda, L, 128, seed=1)
    L.free()


@pytest.mark.parametrize("H,I,group", [(384, 160, 32), (320, 192, 64)])
def test_gemm_layer_ragged(cuda, H, I, group):
    # token blocks and weight-row blocks ragged (100 tokens; I = 160 leaves a
    # 32-row gate/up block, H = 320 a 64-row down block); group 64 scales
    L = DeviceLayer(cuda, H=H, I=I, E=8, k=3, group=group, seed=22, router_std=0.05)
    _layer_vs_oracle(cuda, L, 100, seed=2)
    L.free()


def test_gemm_layer_config3(cuda):
    # 2048 tokens through the Qwen3-30B-A3B-shape layer with
    # the router logits biased by a Zipf(1.1) per-expert offset (v_e += -1.1 ln
    # rank_e over a seeded ranking), so the top expert takes ~23% of the picks.
    # The oracle checks every one of the 2048 tokens (given the same logits),
    # so every expert's last, ragged 128-token tile is covered, the many small
    # tail experts' included.
    T, E = 2048, 128
    L = DeviceLayer(cuda, H=2048, I=768, E=E, k=8, group=32, seed=23)
    x = lp.synth_f32_bf16(T * 2048, 1.0, 3, 1).reshape(T, 2048)
    logits = np.stack([O.router_logits(L.router_w, x[t], E, 2048) for t in range(T)])
    rank = np.random.default_rng(3).permutation(E) + 1
    logits = (logits + (-1.1 * np.log(rank)).astype(np.float32)).astype(np.float32)
    _layer_vs_oracle(cuda, L, T, seed=3, logits=logits, sample=None)
    ids = np.stack([O.top_k_softmax(logits[t], 8, True)[0] for t in range(T)])
    counts = np.bincount(ids.ravel(), minlength=E)
    assert counts.max() > T // 2 and counts.min() < 64 and (counts % 128 != 0).sum() > 64   # skewed, ragged
    L.free()


def h16_images(x: np.ndarray, ngp: int) -> tuple[np.ndarray, np.ndarray]:
    """Restatement of the prefill GEMM's fp16 token images: per row e =
    frexp(max |x|) - 15 (0 for a zero row), x 2^-e rounded to fp16, padded to
    ngp 32-column sub-groups, each 16-byte word holding columns 8 j + (0, 4,
    1, 5, 2, 6, 3, 7) of its sub-group."""
    T, H = x.shape
    m = np.abs(x).max(axis=1)
    e = np.where(m > 0, np.frexp(m)[1] - 15, 0).astype(np.int32)
    xp = np.zeros((T, 32 * ngp), np.float32)
    xp[:, :H] = x
    h = np.ldexp(xp.astype(np.float64), -e[:, None]).astype(np.float16)
    order = np.array([0, 4, 1, 5, 2, 6, 3, 7])
    h = h.reshape(T, ngp, 4, 8)[:, :, :, order].reshape(T, ngp * 32)
    return h.view(np.uint8), e


def test_route_f16_images(cuda):
    # Routing a large batch (T > 64) writes x's fp16 images for the prefill
    # GEMM: byte-exact against h16_images, zero padding sub-groups (H = 320:
    # ten sub-groups, twelve in the image), each row's exponent in xexp; rows
    # scaled by powers of ten (and one zero row) move the exponent.
    T, H = 100, 320
    L = DeviceLayer(cuda, H=H, I=192, E=8, k=3, group=32, seed=24, router_std=0.05)
    x = np.random.default_rng(5).standard_normal((T, H)).astype(np.float32)
    x *= (10.0 ** np.random.default_rng(6).integers(-6, 7, T)).astype(np.float32)[:, None]
    x[3] = 0.0
    lay = lp.ws_layout(L.desc, T)
    assert lay.tiles != lay.actimg, "this shape must take the GEMM path"
    ws = cuda.alloc_device(lay.total)
    dx = cuda.upload(x)
    L.layer.route(dx, T, ws)
    cuda.sync()
    img = cuda.download(ws + lay.xf, (T, 64 * 12), np.uint8)
    xexp = cuda.download(ws + lay.xexp, (T,), np.int32)
    for p in (ws, dx):
        cuda.free_device(p)
    L.free()
    want, we = h16_images(x, 12)
    assert np.array_equal(xexp, we)
    assert np.array_equal(img, want)
    assert np.all(img[:, 64 * 10:] == 0) and np.all(img[3] == 0)
