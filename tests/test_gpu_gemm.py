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


def _bf16_rne(v: np.ndarray) -> np.ndarray:
    b = v.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint32)


def _bf16_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def test_route_bf16_images(cuda):
    # Routing a large batch (T > 64) writes x's bf16 images for the prefill
    # GEMM: per 32-column sub-group the parts hi = bf16(x), lo = bf16(x - hi) in
    # fragment order (word w of 16-byte quarter d pairs columns 8d + w and
    # 8d + w + 4), the seed -136 sum(hi) - 136 sum(lo) and 0, zero padding
    # sub-groups (H = 320: ten sub-groups, twelve in the image), and each
    # token's lo flag (tokens of even index bf16-valued: flag 0).
    T, H = 100, 320
    L = DeviceLayer(cuda, H=H, I=192, E=8, k=3, group=32, seed=24, router_std=0.05)
    x = np.random.default_rng(5).standard_normal((T, H)).astype(np.float32)
    x[0::2] = _bf16_f32(_bf16_rne(x[0::2]))
    lay = lp.ws_layout(L.desc, T)
    assert lay.tiles != lay.actimg, "this shape must take the GEMM path"
    ws = cuda.alloc_device(lay.total)
    dx = cuda.upload(x)
    L.layer.route(dx, T, ws)
    cuda.sync()
    ib = 136 * 12
    img = cuda.download(ws + lay.xf, (T, ib), np.uint8)
    xlo = cuda.download(ws + lay.xlo, (T,), np.int32)
    for p in (ws, dx):
        cuda.free_device(p)
    L.free()
    ngp = 12
    xp = np.zeros((T, 32 * ngp), np.float32)
    xp[:, :H] = x
    hi = _bf16_rne(xp)
    lo = _bf16_rne(xp - _bf16_f32(hi))
    # fragment order: within each 8-column quarter, word w = col w | col w + 4 << 16
    def words(p):
        q = p.reshape(T, ngp, 4, 2, 4)  # [t, g, d, half, w]
        return (q[:, :, :, 0, :] | (q[:, :, :, 1, :] << 16)).astype(np.uint32).reshape(T, ngp * 16)
    got_hi = img[:, :ngp * 64].copy().view(np.uint32)
    got_lo = img[:, ngp * 64:ngp * 128].copy().view(np.uint32)
    assert np.array_equal(got_hi, words(hi))
    assert np.array_equal(got_lo, words(lo))
    seeds = img[:, ngp * 128:].copy().view(np.float32).reshape(T, ngp, 2)
    shi = _bf16_f32(hi).reshape(T, ngp, 32).astype(np.float64).sum(axis=2)
    slo = _bf16_f32(lo).reshape(T, ngp, 32).astype(np.float64).sum(axis=2)
    want = -136.0 * shi - 136.0 * slo
    scale = 136.0 * np.abs(_bf16_f32(hi)).reshape(T, ngp, 32).astype(np.float64).sum(axis=2) + 1e-30
    assert np.all(np.abs(seeds[:, :, 0] - want) <= 4e-6 * scale)
    assert np.all(seeds[:, :, 1] == 0.0)
    assert np.all(seeds[:, 10:, 0] == 0.0)
    assert np.array_equal(xlo, (np.arange(T) % 2).astype(np.int32))
