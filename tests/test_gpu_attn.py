"""The rest of the decode step (decode.cu) and MLA absorbed decode (mla.cu) on
the GPU against the oracle's CPU forms, with the reference's own check
(worst |got - want| / max(|want|, 1), kernels_bench.rs:48-58) and tolerances
(kernels_bench.rs:60-351), at the reference's test shapes and at model
shapes (Qwen3-30B-A3B attention; config 5's MLA: 16 heads, kv_lora 512,
rope 64, context 4096, batch 1 and 16)."""
import numpy as np
import pytest

import llmpager_amd as lp
import _oracle as O
from _gpu import worst_rel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K(cuda):
    return lp.Kernels(cuda)


def _rnd(rng, n):
    return ((rng.random(n) - 0.5) * 2.0).astype(np.float32)


def _bf16(x):
    return ((np.asarray(x, np.float32).view(np.uint32) + 0x8000) >> 16).astype(np.uint16)


def _free(cuda, *ps):
    for p in ps:
        cuda.free_device(p)


@pytest.mark.parametrize("rows,n", [(1, 2048), (8, 128), (32, 4096)])
def test_rmsnorm(cuda, K, rows, n):
    rng = np.random.default_rng(rows)
    x, w = _rnd(rng, rows * n), _rnd(rng, n)
    dx, dw, dy = cuda.upload(x), cuda.upload(w), cuda.alloc_device(rows * n * 4)
    K.rmsnorm(dx, dw, dy, rows, n, 1e-6)
    assert worst_rel(cuda.download(dy, (rows * n,), np.float32), O.rmsnorm(x, w, rows, n, 1e-6)) <= 1e-4
    K.rmsnorm(dx, dw, dx, rows, n, 1e-6)  # in place (the per-head q/k norm)
    assert worst_rel(cuda.download(dx, (rows * n,), np.float32), O.rmsnorm(x, w, rows, n, 1e-6)) <= 1e-4
    _free(cuda, dx, dw, dy)


def test_scale_add_bf16_row_strided_copy(cuda, K):
    rng = np.random.default_rng(9)
    a, b = _rnd(rng, 500), _rnd(rng, 500)
    da, db = cuda.upload(a), cuda.upload(b)
    K.scale_add(da, db, 0.375, 500)
    assert worst_rel(cuda.download(da, (500,), np.float32), O.scale_add(a, b, 0.375)) <= 1e-5
    table = _bf16(_rnd(rng, 10 * 64))
    dt, do = cuda.upload(table), cuda.alloc_device(64 * 4)
    K.bf16_row(dt, 3, 64, do)
    assert np.array_equal(cuda.download(do, (64,), np.float32), O.bf16_row(table, 3, 64))
    src = _rnd(rng, 3 * 16)
    dsrc, ddst = cuda.upload(src), cuda.upload(np.zeros(3 * 8, np.float32))
    K.strided_copy(dsrc, 16, 0, ddst, 8, 2, 3, 5)
    want = O.strided_copy(src, 16, 0, np.zeros(3 * 8, np.float32), 8, 2, 3, 5)
    assert np.array_equal(cuda.download(ddst, (24,), np.float32), want)
    _free(cuda, da, db, dt, do, dsrc, ddst)


@pytest.mark.parametrize("f16", [False, True])
def test_kv_append(cuda, K, f16):
    rng = np.random.default_rng(10)
    kvh, hd, ms, pos = 4, 128, 64, 37
    k, v = _rnd(rng, kvh * hd), _rnd(rng, kvh * hd)
    dt = np.uint16 if f16 else np.float32
    kc0 = np.zeros(kvh * ms * hd, dt)
    dk, dv, dkc, dvc = cuda.upload(k), cuda.upload(v), cuda.upload(kc0), cuda.upload(kc0)
    K.kv_append(dk, dv, dkc, dvc, kvh, hd, pos, ms, f16)
    wk, wv = O.kv_append(k, v, kc0, kc0, kvh, hd, pos, ms, f16)
    assert np.array_equal(cuda.download(dkc, kc0.shape, dt), wk)
    assert np.array_equal(cuda.download(dvc, kc0.shape, dt), wv)
    _free(cuda, dk, dv, dkc, dvc)


@pytest.mark.parametrize("heads,hd,pos,base", [(4, 16, 7, 1e6), (32, 128, 4000, 1e6), (4, 128, 1, 1e4)])
def test_rope(cuda, K, heads, hd, pos, base):
    rng = np.random.default_rng(pos)
    x = _rnd(rng, heads * hd)
    dx = cuda.upload(x)
    K.rope(dx, heads, hd, pos, base)
    # the reference's tolerance (kernels_bench.rs:189-191): at large positions
    # one ulp of powf moves the fp32 angle pos * freq by ~pos * 2^-24 rad, so
    # two correct libraries differ by ~1e-4 there
    tol = 1e-4 if pos < 100 else 5e-3
    assert worst_rel(cuda.download(dx, (heads * hd,), np.float32), O.rope(x, heads, hd, pos, base)) <= tol
    _free(cuda, dx)


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("heads,kvh,hd,seq,ms", [(4, 2, 16, 9, 16), (32, 4, 128, 3000, 4096), (8, 8, 64, 1, 8)])
def test_attn_decode(cuda, K, f16, heads, kvh, hd, seq, ms):
    rng = np.random.default_rng(seq)
    scale = 1.0 / np.sqrt(hd)
    q = _rnd(rng, heads * hd) * 2
    k, v = _rnd(rng, kvh * ms * hd), _rnd(rng, kvh * ms * hd)
    if f16:
        k, v = k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
    dq, dk, dv = cuda.upload(q), cuda.upload(k), cuda.upload(v)
    dout, dscr = cuda.alloc_device(heads * hd * 4), cuda.alloc_device(heads * ms * 4)
    K.attn_decode(dq, dk, dv, dout, dscr, heads, kvh, hd, seq, ms, scale, f16)
    want = O.attn_decode(q, k, v, heads, kvh, hd, seq, ms, scale, f16)
    assert worst_rel(cuda.download(dout, (heads * hd,), np.float32), want) <= 1e-3
    _free(cuda, dq, dk, dv, dout, dscr)


def test_mla_rope(cuda, K):
    rng = np.random.default_rng(11)
    nv, stride, off, half, pos, msc = 3, 20, 4, 6, 9, 1.25
    x = _rnd(rng, nv * stride)
    fr = (0.5 ** np.arange(half) * 0.3).astype(np.float32)
    dx, df = cuda.upload(x), cuda.upload(fr)
    K.mla_rope(dx, nv, stride, off, half, pos, df, msc)
    want = O.mla_rope(x, nv, stride, off, half, pos, fr, msc)
    assert worst_rel(cuda.download(dx, (nv * stride,), np.float32), want) <= 1e-4
    # config 5's q rope slice: 16 heads of [nope 128 | rope 64], position 4095
    nv, stride, off, half, pos = 16, 192, 128, 32, 4095
    x = _rnd(rng, nv * stride)
    fr = (10000.0 ** (-np.arange(half) * 2.0 / 64)).astype(np.float32)
    dx2, df2 = cuda.upload(x), cuda.upload(fr)
    K.mla_rope(dx2, nv, stride, off, half, pos, df2, 1.0)
    want = O.mla_rope(x, nv, stride, off, half, pos, fr, 1.0)
    assert worst_rel(cuda.download(dx2, (nv * stride,), np.float32), want) <= 1e-4
    _free(cuda, dx, df, dx2, df2)


@pytest.mark.parametrize("heads,qk,cd,seq,ms", [(4, 24, 16, 7, 12), (16, 576, 512, 2000, 4096)])
def test_mla_attn_decode(cuda, K, heads, qk, cd, seq, ms):
    rng = np.random.default_rng(seq)
    scale = 0.31 if qk == 24 else 0.0722
    q = _rnd(rng, heads * qk)
    cache = _rnd(rng, ms * qk)
    dq, dc = cuda.upload(q), cuda.upload(cache)
    dctx, dscr = cuda.alloc_device(heads * cd * 4), cuda.alloc_device(heads * ms * 4)
    K.mla_attn_decode(dq, dc, dctx, dscr, heads, qk, cd, seq, ms, scale)
    want = O.mla_attn_decode(q, cache[:seq * qk], heads, qk, cd, seq, scale)
    assert worst_rel(cuda.download(dctx, (heads * cd,), np.float32), want) <= 1e-3
    _free(cuda, dq, dc, dctx, dscr)


@pytest.mark.parametrize("rows,cols,batch,xs", [(16, 32, 3, 0), (512, 128, 16, 192), (13, 37, 2, 37)])
def test_bf16_gemv_batch(cuda, K, rows, cols, batch, xs):
    rng = np.random.default_rng(rows)
    w = _bf16(_rnd(rng, batch * rows * cols))
    x = _rnd(rng, max(1, (batch - 1) * xs + cols))
    ys = rows + 3
    dw, dx = cuda.upload(w), cuda.upload(x)
    dy = cuda.upload(np.zeros((batch - 1) * ys + rows, np.float32))
    K.bf16_gemv_batch(dw, rows * cols, dx, xs, dy, ys, rows, cols, batch)
    got = cuda.download(dy, ((batch - 1) * ys + rows,), np.float32)
    want = O.bf16_gemv_batch(w, rows * cols, x, xs, ys, rows, cols, batch)
    assert worst_rel(got, want) <= 1e-4
    _free(cuda, dw, dx, dy)


def _mla_batch(cuda, K, heads, qk, cd, seqs, ms, scale, qstd, seed, device_seqs=None):
    rng = np.random.default_rng(seed)
    B = len(seqs)
    q = (rng.standard_normal(B * heads * qk) * qstd).astype(np.float32)
    cache = _bf16(rng.standard_normal(B * ms * qk).astype(np.float32))   # N(0, 1) latent KV
    dq, dc = cuda.upload(q), cuda.upload(cache)
    dsl = cuda.upload(np.asarray(seqs if device_seqs is None else device_seqs, np.int32))
    dctx = cuda.alloc_device(B * heads * cd * 4)
    ws = cuda.alloc_device(K.mla_batch_ws_bytes(B, cd, ms))
    K.mla_attn_decode_batch(dq, dc, ms * qk * 2, dsl, dctx, ws, B, heads, qk, cd, ms, scale)
    got = cuda.download(dctx, (B, heads * cd), np.float32)
    for b, sq in enumerate(seqs):
        want = O.mla_attn_decode(q[b * heads * qk:(b + 1) * heads * qk], cache[b * ms * qk:b * ms * qk + sq * qk],
                                 heads, qk, cd, sq, scale, bf16=True)
        err = worst_rel(got[b], want)
        assert err <= 1e-3, (b, sq, err)
    _free(cuda, dq, dc, dsl, dctx, ws)


def test_mla_batch_small_shapes(cuda, K):
    # 4 heads (padded to the 16-row tile), qk 96, c_dim 64; ragged lengths
    # (one position, a partial chunk, several chunks)
    _mla_batch(cuda, K, 4, 96, 64, [1, 63, 200], 256, 0.2, 1.0, 1)


def test_mla_batch_lengths_past_the_cache_are_clamped(cuda, K):
    # device lengths above max_seq (256) read only the sequence's own 256
    # rows: the result is that of a full-length sequence (unclamped, the
    # first two would also read the following sequences' rows)
    _mla_batch(cuda, K, 4, 96, 64, [256, 256, 63], 256, 0.2, 1.0, 2, device_seqs=[1000, 257, 63])


@pytest.mark.parametrize("B,qstd", [(1, 0.05), (1, 1.0), (16, 0.05), (16, 1.0)])
def test_mla_batch_config5(cuda, K, B, qstd):
    # config 5: 16 heads, [kv_lora 512 | rope 64] latent rows, context 4096;
    # at B = 16 the sequences' lengths vary (full, ragged, one position)
    seqs = [4096] if B == 1 else [4096, 4095, 1, 64, 65, 2048, 3000, 4096, 17, 1000, 4032, 129, 4096, 511, 2, 3333]
    _mla_batch(cuda, K, 16, 576, 512, seqs, 4096, 0.0722, qstd, 100 + B)
