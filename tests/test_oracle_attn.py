"""Pins for the oracle's decode-step and MLA restatements (oracle/lp_oracle.c,
the CPU forms of crates/llmpager-bench/src/kernels_bench.rs:60-351): each is
checked against float64 closed forms written independently here with numpy
(softmax attention, rotations, normalisation), plus IEEE half rounding
against numpy's float16.  A wrong head mapping, rotation pairing, scale or
softmax term fails one of them."""
import numpy as np
import pytest

import _oracle as O


def _rnd(rng, n):
    return ((rng.random(n) - 0.5) * 2.0).astype(np.float32)


def _bf16(x):
    # round-half-up bf16 bits, the reference's own test helper
    # (kernels_bench.rs:16-18)
    return ((x.astype(np.float32).view(np.uint32) + 0x8000) >> 16).astype(np.uint16)


def _bf16_val(h):
    return (h.astype(np.uint32) << 16).view(np.float32)


def test_f16_rne_matches_numpy():
    rng = np.random.default_rng(0)
    bits = np.concatenate([rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32),
                           np.arange(0x33000000, 0x39000000, 4099, dtype=np.uint32),   # subnormal edge
                           np.arange(0x477F0000, 0x47800000, 7, dtype=np.uint32)])     # overflow edge
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    want = x.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16_rne(float(v)) for v in x[:60000]], np.uint16)
    assert np.array_equal(got, want[:60000])


def test_rmsnorm_closed_form():
    rng = np.random.default_rng(1)
    rows, n = 8, 128
    x, w = _rnd(rng, rows * n), _rnd(rng, n)
    got = O.rmsnorm(x, w, rows, n, 1e-6).reshape(rows, n)
    xd = x.astype(np.float64).reshape(rows, n)
    want = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6) * w.astype(np.float64)
    assert np.allclose(got, want, rtol=2e-6, atol=1e-6)


def test_scale_add_kv_append_row_copy():
    rng = np.random.default_rng(2)
    a, b = _rnd(rng, 500), _rnd(rng, 500)
    assert np.allclose(O.scale_add(a, b, 0.375), a.astype(np.float64) + 0.375 * b, rtol=1e-6, atol=1e-7)
    kvh, hd, ms, pos = 4, 16, 8, 5
    k, v = _rnd(rng, kvh * hd), _rnd(rng, kvh * hd)
    kc, vc = O.kv_append(k, v, np.zeros(kvh * ms * hd, np.float32), np.zeros(kvh * ms * hd, np.float32),
                         kvh, hd, pos, ms, False)
    want = np.zeros((kvh, ms, hd), np.float32)
    want[:, pos, :] = k.reshape(kvh, hd)
    assert np.array_equal(kc.reshape(kvh, ms, hd), want)
    kc, vc = O.kv_append(k, v, np.zeros(kvh * ms * hd, np.uint16), np.zeros(kvh * ms * hd, np.uint16),
                         kvh, hd, pos, ms, True)
    assert np.array_equal(vc.reshape(kvh, ms, hd)[:, pos, :], v.reshape(kvh, hd).astype(np.float16).view(np.uint16))
    table = _bf16(_rnd(rng, 10 * 64))
    assert np.array_equal(O.bf16_row(table, 3, 64), _bf16_val(table[3 * 64:4 * 64]))
    src = _rnd(rng, 3 * 16)
    got = O.strided_copy(src, 16, 0, np.zeros(3 * 8, np.float32), 8, 2, 3, 5)
    want = np.zeros((3, 8), np.float32)
    want[:, 2:7] = src.reshape(3, 16)[:, :5]
    assert np.array_equal(got.reshape(3, 8), want)


def test_rope_closed_form():
    rng = np.random.default_rng(3)
    heads, hd, pos, base = 4, 16, 7, 1e6
    x = _rnd(rng, heads * hd)
    got = O.rope(x, heads, hd, pos, base).reshape(heads, hd)
    xd = x.astype(np.float64).reshape(heads, hd)
    i = np.arange(hd // 2)
    ang = pos * base ** (-2.0 * i / hd)
    c, s = np.cos(ang), np.sin(ang)
    want = np.concatenate([xd[:, :hd // 2] * c - xd[:, hd // 2:] * s, xd[:, :hd // 2] * s + xd[:, hd // 2:] * c], 1)
    assert np.allclose(got, want, atol=2e-6)


def _softmax_attn(q, k, v, scale):
    s = (k @ q) * scale
    e = np.exp(s - s.max())
    return (e / e.sum()) @ v


@pytest.mark.parametrize("f16", [False, True])
def test_attn_decode_closed_form(f16):
    rng = np.random.default_rng(4)
    heads, kvh, hd, seq, ms = 8, 2, 16, 9, 16
    scale = 1.0 / np.sqrt(hd)
    q = _rnd(rng, heads * hd)
    k, v = _rnd(rng, kvh * ms * hd), _rnd(rng, kvh * ms * hd)
    if f16:
        kc, vc = k.astype(np.float16), v.astype(np.float16)
        kw, vw = kc.astype(np.float64), vc.astype(np.float64)
        kc, vc = kc.view(np.uint16), vc.view(np.uint16)
    else:
        kc, vc, kw, vw = k, v, k.astype(np.float64), v.astype(np.float64)
    got = O.attn_decode(q, kc, vc, heads, kvh, hd, seq, ms, scale, f16).reshape(heads, hd)
    kw, vw = kw.reshape(kvh, ms, hd), vw.reshape(kvh, ms, hd)
    for h in range(heads):
        g = h // (heads // kvh)
        want = _softmax_attn(q[h * hd:(h + 1) * hd].astype(np.float64), kw[g, :seq], vw[g, :seq], scale)
        assert np.allclose(got[h], want, rtol=1e-5, atol=1e-6), h


def test_mla_rope_closed_form():
    rng = np.random.default_rng(5)
    nv, stride, off, half, pos, ms = 3, 20, 4, 6, 9, 1.25
    x = _rnd(rng, nv * stride)
    fr = (0.5 ** np.arange(half) * 0.3).astype(np.float32)
    got = O.mla_rope(x, nv, stride, off, half, pos, fr, ms).reshape(nv, stride)
    want = x.astype(np.float64).reshape(nv, stride).copy()
    ang = pos * fr.astype(np.float64)
    c, s = np.cos(ang) * ms, np.sin(ang) * ms
    x1, x2 = want[:, off:off + 2 * half:2].copy(), want[:, off + 1:off + 2 * half:2].copy()
    want[:, off:off + 2 * half:2] = x1 * c - x2 * s
    want[:, off + 1:off + 2 * half:2] = x1 * s + x2 * c
    assert np.allclose(got, want, atol=2e-6)


@pytest.mark.parametrize("bf16", [False, True])
def test_mla_attn_decode_closed_form(bf16):
    rng = np.random.default_rng(6)
    heads, qk, cd, seq = 4, 24, 16, 7
    scale = 0.31
    q = _rnd(rng, heads * qk)
    cache = _rnd(rng, seq * qk)
    if bf16:
        cb = _bf16(cache)
        cw = _bf16_val(cb).astype(np.float64).reshape(seq, qk)
        cache = cb
    else:
        cw = cache.astype(np.float64).reshape(seq, qk)
    got = O.mla_attn_decode(q, cache, heads, qk, cd, seq, scale, bf16=bf16).reshape(heads, cd)
    for h in range(heads):
        want = _softmax_attn(q[h * qk:(h + 1) * qk].astype(np.float64), cw, cw[:, :cd], scale)
        assert np.allclose(got[h], want, rtol=1e-5, atol=1e-6), h


def test_bf16_gemv_batch_closed_form():
    rng = np.random.default_rng(7)
    rows, cols, batch = 16, 32, 3
    w = _bf16(_rnd(rng, batch * rows * cols))
    x = _rnd(rng, cols)
    got = O.bf16_gemv_batch(w, rows * cols, x, 0, rows, rows, cols, batch).reshape(batch, rows)
    want = _bf16_val(w).astype(np.float64).reshape(batch, rows, cols) @ x.astype(np.float64)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("rows,cols", [(7, 8), (33, 2048), (5, 4096), (3, 37)])
def test_bf16_gemv_closed_form(rows, cols):
    # y = W x against float64 (each product of a bf16 weight and an fp32
    # value is exact in float64), within the fp32 chain's rounding bound
    # n * 2^-24 * sum |w x|; then the special cases that are exact in fp32
    rng = np.random.default_rng(rows * cols)
    w = _bf16(_rnd(rng, rows * cols))
    x = _rnd(rng, cols)
    got = O.bf16_gemv(w, x, rows, cols).astype(np.float64)
    wf = _bf16_val(w).astype(np.float64).reshape(rows, cols)
    want = wf @ x.astype(np.float64)
    bound = cols * 2.0 ** -24 * (np.abs(wf) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(got - want) <= bound + 1e-30)
    # a one-hot row picks one column exactly; a zero row gives 0; a row of
    # 1.0 over small integers sums exactly
    w2 = np.zeros((3, cols), np.uint16)
    w2[0, cols // 2] = 0x3F80  # bf16 1.0
    w2[2, :] = 0x3F80
    xi = (np.arange(cols) % 7).astype(np.float32)
    y2 = O.bf16_gemv(w2.reshape(-1), xi, 3, cols)
    assert y2[0] == xi[cols // 2] and y2[1] == 0.0 and y2[2] == float(xi.sum())
