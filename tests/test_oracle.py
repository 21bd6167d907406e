"""Pins the CPU oracle before it is trusted as the checker.

Sources of truth, strongest first: the reference's own known-answer tests
(ported here with their file:line), exhaustive or strided comparison with the
library the reference calls (glibc expf), closed forms, and brute force on
small inputs.  Each check is chosen so that a plausible slip in the oracle
(a dropped term, a flipped sort, an off-by-one nibble) fails it."""
import math
import struct

import numpy as np
import pytest

import _oracle as O


def pseudo(n: int, seed: int) -> np.ndarray:
    """quant.rs:199-209: xorshift values in [-0.1, 0.1)."""
    s = max(seed, 1)
    out = np.empty(n, np.float32)
    M = (1 << 64) - 1
    for i in range(n):
        s ^= (s << 13) & M
        s ^= s >> 7
        s ^= (s << 17) & M
        out[i] = np.float32((s >> 11) / float(1 << 53) * 2.0 - 1.0) * np.float32(0.1)
    return out


# ---- routing: reference known answers ----------------------------------------------

def test_topk_renorm_known_answer():
    # decode.rs:786-793
    ids, w = O.top_k_softmax(np.array([0, 1, 2, 3], np.float32), 2, True)
    assert list(ids) == [3, 2]
    assert abs(float(w[0]) + float(w[1]) - 1.0) < 1e-6
    assert w[0] > w[1]


def test_sigmoid_bias_affects_selection_not_weights():
    # kimi.rs:1219-1233
    ids, w = O.sigmoid_topk(np.array([2.0, -2.0, 1.0, -3.0], np.float32),
                            np.array([0.0, 0.0, 5.0, 0.0], np.float32), 2, True, 2.0, 0.0)
    assert list(ids) == [2, 0]
    s0 = 1.0 / (1.0 + math.exp(-2.0))
    s2 = 1.0 / (1.0 + math.exp(-1.0))
    assert abs(float(w[0]) - s2 / (s0 + s2) * 2.0) < 1e-5


def test_sigmoid_min_weight_drops_tail():
    # kimi.rs:1235-1241
    ids, w = O.sigmoid_topk(np.array([4.0, 4.0, -6.0], np.float32), np.zeros(3, np.float32),
                            3, True, 1.0, 0.05)
    assert len(ids) == 2


# ---- routing: brute force against an independent float32 restatement --------------

def _softmax_topk_brute(logits: np.ndarray, k: int, renorm: bool):
    """Same semantics written the other way round: float32 numpy scalars, the
    exponentials taken from glibc one by one, and a full sort with an explicit
    (p descending, id ascending) key -- no insertion sort."""
    f = np.float32
    m = f(-3.4028234663852886e38)
    for v in logits:
        m = max(m, f(v))
    e = [f(O.expf(float(f(v) - m))) for v in logits]
    z = f(-0.0)
    for v in e:
        z = f(z + v)
    p = [f(v / z) for v in e]
    order = sorted(range(len(p)), key=lambda i: (-float(p[i]), i))[:k]
    w = [p[i] for i in order]
    if renorm:
        s = f(-0.0)
        for v in w:
            s = f(s + v)
        w = [f(v / s) for v in w]
    return np.array(order, np.int32), np.array(w, np.float32)


@pytest.mark.parametrize("E,k", [(4, 2), (8, 2), (16, 5), (128, 8)])
def test_top_k_softmax_brute(E, k):
    rng = np.random.default_rng(E + k)
    rows = [rng.standard_normal(E).astype(np.float32) * s for s in (0.01, 1, 10)]
    t = rng.standard_normal(E).astype(np.float32)
    t[: min(4, E)] = 7.0  # exact ties
    rows.append(t)
    rows.append(np.zeros(E, np.float32))
    for r in rows:
        for renorm in (False, True):
            ids, w = O.top_k_softmax(r, k, renorm)
            bi, bw = _softmax_topk_brute(r, k, renorm)
            assert np.array_equal(ids, bi)
            assert np.array_equal(w.view(np.uint32), bw.view(np.uint32))


def test_sigmoid_topk_brute_and_negative_zero_tie():
    f = np.float32
    rng = np.random.default_rng(3)
    E, k = 32, 6
    for trial in range(20):
        lg = (rng.standard_normal(E) * 2).astype(np.float32)
        bias = (rng.standard_normal(E) * 0.3).astype(np.float32)
        ids, w = O.sigmoid_topk(lg, bias, k, True, 2.5, 0.0)
        s = [f(1.0) / f(f(1.0) + f(O.expf(float(-v)))) for v in lg]
        key = [f(s[i] + bias[i]) for i in range(E)]
        order = sorted(range(E), key=lambda i: (-float(key[i]), i))[:k]
        tot = f(-0.0)
        for i in order:
            tot = f(tot + s[i])
        want = [f(f(s[i] / tot) * f(2.5)) for i in order]
        assert list(ids) == order
        assert np.array_equal(w, np.array(want, np.float32))
    # -0.0 and +0.0 keys rank as equal: the lower id stays first
    lg = np.zeros(4, np.float32)
    s0 = np.float32(0.5)
    bias = np.array([-0.0, 0.0, -s0, -s0], np.float32)
    bias[0] = -s0
    bias[1] = -s0
    ids, _ = O.sigmoid_topk(lg, bias, 4, False, 1.0, 0.0)
    assert list(ids) == [0, 1, 2, 3]


# ---- expf: the library the reference calls --------------------------------------------

def test_expf_is_libm():
    for x in (0.0, 1.0, -1.0, -87.0, -103.9, 88.5, -0.5):
        assert O.expf(x) == np.float32(math.exp(x)) or abs(O.expf(x) / math.exp(x) - 1) < 1e-7


# ---- q4 format: reference tests quant.rs:196-276 -----------------------------------------

def test_g32_round_trip_and_store_group():
    # quant.rs:212-244
    rows, cols, group = 4, 128, 32
    src = pseudo(rows * cols, 9)
    buf, max_err = O.q4_quantize(src, rows, cols, group)
    back = O.q4_dequantize(buf, rows, cols, group).ravel()
    assert np.all(np.abs(src - back) <= max_err + 1e-6)
    buf2 = np.zeros_like(buf)
    gpr = cols // group
    scales_len = rows * gpr * 2
    for r in range(rows):
        for g in range(gpr):
            sidx = (r * gpr + g) * 2
            scale = O.f16_to_f32(int(buf[sidx]) | (int(buf[sidx + 1]) << 8))
            base = scales_len + r * cols // 2 + g * group // 2
            qs = np.zeros(group, np.uint8)
            qs[0::2] = buf[base:base + group // 2] & 0x0F
            qs[1::2] = buf[base:base + group // 2] >> 4
            O.q4_store_group(buf2, rows, cols, group, r, g, scale, qs)
    assert np.array_equal(buf, buf2)


def test_round_trip_error_bounded():
    # quant.rs:247-260
    rows, cols = 8, 256
    src = pseudo(rows * cols, 3)
    buf, max_err = O.q4_quantize(src, rows, cols, 64)
    back = O.q4_dequantize(buf, rows, cols, 64).ravel()
    assert np.all(np.abs(src - back) <= max_err + 1e-6)
    assert max_err < 0.1 / 14.0 * 1.1


def test_f16_helpers():
    # quant.rs:263-268
    for x in (0.0, 1.0, -1.0, 0.5, 65504.0, 1e-8, 3.14159):
        y = O.f16_to_f32(O.f32_to_f16_ref(x))
        assert abs(x - y) <= max(abs(x) * 0.001, 1e-7)


def test_rejects_bad_dims():
    # quant.rs:271-275
    with pytest.raises(ValueError):
        O.q4_quantize(np.zeros(10, np.float32), 1, 10, 64)


def test_f16_encoder_carry_quirk():
    # quant.rs:170 ORs the rounding carry into the exponent: 1.9999 -> 1.0,
    # 7.9999 -> 4.0 (known answers of an independent restatement); ties half-up.
    assert O.f32_to_f16_ref(1.9999) == 0x3C00
    assert O.f32_to_f16_ref(7.9999) == 0x4400
    assert O.f32_to_f16_ref(0.0019531) == 0x1400
    # Against IEEE round-to-nearest-even: within one unit (ties go half-up),
    # except where rounding carries into the next binade: there the OR keeps
    # the exponent when its low bit was already set, so the result is either
    # the IEEE value or the same mantissa one binade lower.
    rng = np.random.default_rng(0)
    carries = 0
    for v in rng.uniform(1e-3, 100, 20000).astype(np.float32):
        got = int(O.f32_to_f16_ref(float(v)))
        ieee = int(np.float16(v).view(np.uint16))
        own_exp = (int(np.float32(v).view(np.uint32)) >> 23) - 127 + 15
        if (ieee & 0x3FF) == 0 and (ieee >> 10) == own_exp + 1:
            assert got in (ieee, ieee - 0x400)
            carries += got != ieee
        else:
            assert abs(got - ieee) <= 1
    assert carries > 0


def test_f16_decoder_exhaustive():
    # quant.rs:173-189 is exact: every finite f16 decodes to numpy's value
    for h in range(0x10000):
        e = (h >> 10) & 0x1F
        if e == 0x1F:
            continue
        assert O.f16_to_f32(h) == float(np.array([h], np.uint16).view(np.float16)[0])


# ---- GEMV forms: brute force ---------------------------------------------------------------

@pytest.mark.parametrize("rows,cols,group", [(16, 64, 32), (33, 128, 64), (8, 96, 32)])
def test_q4_gemv_matches_float64_dequant(rows, cols, group):
    rng = np.random.default_rng(rows)
    w = rng.standard_normal(rows * cols).astype(np.float32) * 0.05
    buf, _ = O.q4_quantize(w, rows, cols, group)
    # decode the nibbles independently of the oracle: byte i/2, low nibble even
    gpr = cols // group
    sc = buf[: rows * gpr * 2].view(np.uint16).reshape(rows, gpr).view(np.float16).astype(np.float64)
    data = buf[rows * gpr * 2:].reshape(rows, cols // 2)
    q = np.empty((rows, cols), np.int64)
    q[:, 0::2] = data & 0x0F
    q[:, 1::2] = data >> 4
    wd = (q - 8) * np.repeat(sc, group, axis=1)
    x = rng.standard_normal(cols).astype(np.float32)
    want = wd @ x.astype(np.float64)
    got = O.q4_gemv(buf, x, rows, cols, group)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5)


def test_router_logits_canonical_matches_float64():
    rng = np.random.default_rng(1)
    E, H = 16, 2048
    w = rng.integers(0, 1 << 16, E * H).astype(np.uint16)
    w &= 0xBFFF  # keep magnitudes finite and modest
    x = rng.standard_normal(H).astype(np.float32)
    got = O.router_logits(w, x, E, H)
    wf = (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(E, H)
    want = wf @ x.astype(np.float64)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-4 * np.abs(wf).sum(1).max())


def test_silu_moe_reduce_add_closed_form():
    rng = np.random.default_rng(2)
    g = rng.standard_normal(64).astype(np.float32)
    u = rng.standard_normal(64).astype(np.float32)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(O.silu_mul(g, u), want, rtol=1e-6, atol=1e-7)
    eo = rng.standard_normal((5, 64)).astype(np.float32)
    wt = rng.random(5).astype(np.float32)
    h = rng.standard_normal(64).astype(np.float32)
    want = h.astype(np.float64) + (wt[:, None].astype(np.float64) * eo).sum(0)
    assert np.allclose(O.moe_reduce(eo, wt, h), want, rtol=1e-6, atol=1e-6)
    assert np.array_equal(O.add(g, u), g + u)


# ---- dispatch: invariants and brute force ------------------------------------------------

@pytest.mark.parametrize("T,k,E", [(1, 8, 128), (8, 8, 128), (33, 2, 8), (200, 6, 64)])
def test_dispatch_brute(T, k, E):
    rng = np.random.default_rng(T * k)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    cnt = rng.integers(1, k + 1, T).astype(np.int32)
    perm, gs, inv, uniq = O.moe_dispatch(ids, cnt, T, k, E)
    pairs = sorted(((int(ids[t, j]), t, j) for t in range(T) for j in range(cnt[t])))
    assert [t * k + j for _, t, j in pairs] == list(perm)
    assert list(uniq) == sorted({e for e, _, _ in pairs})
    for e in range(E):
        assert gs[e + 1] - gs[e] == sum(1 for p in pairs if p[0] == e)
    for pos, pk in enumerate(perm):
        assert inv[pk] == pos
    for t in range(T):
        assert all(inv[t * k + j] == -1 for j in range(cnt[t], k))


# ---- whole layer: composition ------------------------------------------------------------

def test_layer_composition_small():
    """lpo_moe_layer equals the composition of the pinned pieces, and the wave
    split of decode.rs:489-531 changes only the grouping of partial sums."""
    import llmpager_amd as lp
    H, I, E, k, g = 128, 64, 8, 2, 32
    span = 16384
    host = lp.synth_blobs(E, span, H, I, g, 4, 0)
    bb = lp.blob_bytes(H, I, g)
    blobs = [host[e * span: e * span + bb] for e in range(E)]
    go, uo, do = lp.blob_offsets(H, I, g)
    rw = lp.synth_bf16(E * H, 0.2, 4, 1)
    desc = dict(hidden=H, inter=I, experts=E, top_k=k, group=g, gating=0, renorm=True,
                router_w=rw, offsets=(go, uo, do))
    T = 3
    x = lp.synth_f32_bf16(T * H, 1.0, 4, 1).reshape(T, H)
    h = lp.synth_f32_bf16(T * H, 1.0, 4, 2).reshape(T, H)
    hout, logits, ids, w, cnt = O.moe_layer(desc, blobs, x, h)
    for t in range(T):
        lg = O.router_logits(rw, x[t], E, H)
        assert np.array_equal(lg, logits[t])
        wi, ww = O.top_k_softmax(lg, k, True)
        assert np.array_equal(wi, ids[t, :cnt[t]])
        ys = []
        for e in wi:
            b = blobs[e]
            gg = O.q4_gemv(b[go:], x[t], I, H, g)
            uu = O.q4_gemv(b[uo:], x[t], I, H, g)
            ys.append(O.q4_gemv(b[do:], O.silu_mul(gg, uu), H, I, g))
        want = O.moe_reduce(np.stack(ys), ww, h[t])
        assert np.array_equal(want, hout[t])
    h1 = O.moe_layer(desc, blobs, x, h, wave=1)[0]
    assert np.allclose(h1, hout, rtol=1e-6, atol=1e-6)


def test_layer_composition_sigmoid_shared():
    """The sigmoid + bias branch with renormalisation, scaling and min_weight,
    plus the always-on shared MLP (kimi.rs:739-779): lpo_moe_layer equals the
    composition of the pinned pieces -- routed picks summed in pick order and
    added once, then the shared MLP's output added unweighted -- at any
    thread count."""
    import llmpager_amd as lp
    H, I, E, k, g = 128, 64, 16, 4, 32
    SI, SG = 128, 64
    span = 16384
    host = lp.synth_blobs(E, span, H, I, g, 6, 0)
    bb = lp.blob_bytes(H, I, g)
    blobs = [host[e * span: e * span + bb] for e in range(E)]
    go, uo, do = lp.blob_offsets(H, I, g)
    sgo, suo, sdo = lp.blob_offsets(H, SI, SG)
    shared = lp.synth_blob(H, SI, SG, 6, 0, 1 << 20)
    rw = lp.synth_bf16(E * H, 0.2, 6, 1)
    bias = (np.random.default_rng(6).standard_normal(E) * 0.3).astype(np.float32)
    scaling, min_w = 2.5, 0.6
    desc = dict(hidden=H, inter=I, experts=E, top_k=k, group=g, gating=O.GATING_SIGMOID, renorm=True,
                routed_scaling=scaling, min_weight=min_w, router_w=rw, router_bias=bias,
                offsets=(go, uo, do))
    sh = dict(blob=shared, inter=SI, group=SG, offsets=(sgo, suo, sdo))
    T = 6
    x = lp.synth_f32_bf16(T * H, 1.0, 6, 1).reshape(T, H)
    h = lp.synth_f32_bf16(T * H, 1.0, 6, 2).reshape(T, H)
    hout, logits, ids, w, cnt = O.moe_layer(desc, blobs, x, h, shared_blob=sh)
    assert (cnt < k).any() and (cnt > 0).all()  # min_weight dropped some picks, not all
    for t in range(T):
        lg = O.router_logits(rw, x[t], E, H)
        assert np.array_equal(lg, logits[t])
        wi, ww = O.sigmoid_topk(lg, bias, k, True, scaling, min_w)
        assert np.array_equal(wi, ids[t, :cnt[t]])
        assert np.array_equal(ww.view(np.uint32), w[t, :cnt[t]].view(np.uint32))
        ys = []
        for e in wi:
            b = blobs[e]
            gg = O.q4_gemv(b[go:], x[t], I, H, g)
            uu = O.q4_gemv(b[uo:], x[t], I, H, g)
            ys.append(O.q4_gemv(b[do:], O.silu_mul(gg, uu), H, I, g))
        want = O.moe_reduce(np.stack(ys), ww, h[t])
        sg = O.q4_gemv(shared[sgo:], x[t], SI, H, SG)
        su = O.q4_gemv(shared[suo:], x[t], SI, H, SG)
        want = O.add(want, O.q4_gemv(shared[sdo:], O.silu_mul(sg, su), H, SI, SG))
        assert np.array_equal(want, hout[t])
    # the shared output is the exact difference a no-shared layer leaves
    h_routed = O.moe_layer(desc, blobs, x, h)[0]
    assert not np.array_equal(h_routed, hout)
    assert np.array_equal(O.moe_layer(desc, blobs, x, h, shared_blob=sh, threads=4)[0], hout)
