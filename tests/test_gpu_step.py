"""A whole decode step (llmpager_amd.step: per layer the attention block,
either as the reference's one launch per kernels.rs call or as the three
fused launches, and the fused MoE layer, then the final norm and the
lm_head) against the oracle's composition of the same functions in the
order of decode.rs:263-363, over several positions; the step recorded once
with lp_graph_capture_begin / lp_graph_capture_end, whose replay equals the
eager step bit for bit; and each fused launch (lp_rmsnorm_gemv,
lp_gemv_add_rmsnorm, lp_attn_fused, lp_attn_block) against the oracle
functions it combines, at the test shapes and at Qwen3-30B-A3B's.

Tolerances: the logits within rel-L2 1e-3 of the oracle's (the MoE layers'
own bound); the fused launches with the reference's check (worst |got -
want| / max(|want|, 1), kernels_bench.rs:48-58) at the bounds its tests
give the kernels they combine: 1e-4 for rmsnorm and bf16_gemv, 1e-3 for
attention (kernels_bench.rs:60-256).  The cache row a fused launch appends
is the fp16 rounding of its own normed, rotated k: within one fp16 step of
the oracle's."""
import numpy as np
import pytest

import llmpager_amd as lp
import _oracle as O
from _gpu import DeviceLayer, rel_l2, worst_rel
from llmpager_amd.step import AttnWeights, DecodeStep, StepShape

pytestmark = pytest.mark.gpu


def _build(cuda, S: StepShape, NL: int, seed: int, fused=None, moe_shape=None):
    rng = np.random.default_rng(seed)
    H, qd, kd = S.hidden, S.heads * S.head_dim, S.kv_heads * S.head_dim
    host, attn, moe, allocs = [], [], [], []

    def up(a):
        p = cuda.upload(np.ascontiguousarray(a))
        allocs.append(p)
        return p
    for l in range(NL):
        w = dict(q=lp.synth_bf16(qd * H, 0.05, seed, 10 * l + 1), k=lp.synth_bf16(kd * H, 0.05, seed, 10 * l + 2),
                 v=lp.synth_bf16(kd * H, 0.05, seed, 10 * l + 3), o=lp.synth_bf16(H * qd, 0.05, seed, 10 * l + 4),
                 input_ln=(1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32),
                 q_norm=(1.0 + 0.1 * rng.standard_normal(S.head_dim)).astype(np.float32),
                 k_norm=(1.0 + 0.1 * rng.standard_normal(S.head_dim)).astype(np.float32),
                 post_ln=(1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32))
        host.append(w)
        attn.append(AttnWeights(**{k: up(v) for k, v in w.items()}))
        ms = moe_shape or dict(I=64, E=8, k=2, group=32, router_std=0.1)
        moe.append(DeviceLayer(cuda, H=H, seed=seed + l, layer=l, **ms))
    embed = lp.synth_bf16(S.vocab * H, 1.0, seed, 900)
    lm = lp.synth_bf16(S.vocab * H, 0.05, seed, 901)
    fn = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    ws_bytes = max(lp.ws_layout(L.desc, 1).total for L in moe)
    ws = cuda.alloc_device(ws_bytes)
    allocs.append(ws)
    step = DecodeStep(cuda, S, attn, [L.layer for L in moe], up(embed), up(fn), up(lm), ws, ws_bytes, fused=fused)
    return step, dict(layers=host, embed=embed, lm=lm, fn=fn), moe, allocs


def _oracle_step(S: StepShape, W: dict, moe, caches, token: int, pos: int) -> np.ndarray:
    H, qd, kd = S.hidden, S.heads * S.head_dim, S.kv_heads * S.head_dim
    h = O.bf16_row(W["embed"], token, H)
    for l, (w, L) in enumerate(zip(W["layers"], moe)):
        hn = O.rmsnorm(h, w["input_ln"], 1, H, S.eps)
        q, k, v = O.bf16_gemv(w["q"], hn, qd, H), O.bf16_gemv(w["k"], hn, kd, H), O.bf16_gemv(w["v"], hn, kd, H)
        q = O.rope(O.rmsnorm(q, w["q_norm"], S.heads, S.head_dim, S.eps), S.heads, S.head_dim, pos, S.rope_theta)
        k = O.rope(O.rmsnorm(k, w["k_norm"], S.kv_heads, S.head_dim, S.eps), S.kv_heads, S.head_dim, pos,
                   S.rope_theta)
        caches[l] = O.kv_append(k, v, caches[l][0], caches[l][1], S.kv_heads, S.head_dim, pos, S.max_seq, S.kv_f16)
        a = O.attn_decode(q, caches[l][0], caches[l][1], S.heads, S.kv_heads, S.head_dim, pos + 1, S.max_seq,
                          1.0 / float(np.sqrt(S.head_dim)), S.kv_f16)
        h = O.add(h, O.bf16_gemv(w["o"], a, H, qd))
        hn = O.rmsnorm(h, w["post_ln"], 1, H, S.eps)
        h = O.moe_layer(L.oracle_desc(), L.oracle_blobs(), hn[None, :], h[None, :].copy(), threads=4)[0][0]
    return O.bf16_gemv(W["lm"], O.rmsnorm(h, W["fn"], 1, H, S.eps), S.vocab, H)


@pytest.mark.parametrize("hd,fused,max_seq,positions", [
    (64, False, 16, (0, 1, 2, 3)),      # the reference's launch sequence
    (128, False, 16, (0, 1, 2, 3)),
    (128, True, 16, (0, 1, 2, 3)),      # fused, one split
    (128, True, 512, (0, 1, 130, 300)),  # fused, split positions merged
])
def test_decode_step_against_oracle_and_graph(cuda, hd, fused, max_seq, positions):
    S = StepShape(hidden=256, heads=4, kv_heads=2, head_dim=hd, vocab=700, max_seq=max_seq)
    step, W, moe, allocs = _build(cuda, S, NL=2, seed=31, fused=fused)
    assert step.fused == fused
    kd = S.kv_heads * S.head_dim
    z = np.zeros(kd * S.max_seq, np.uint16)
    for c in step.kcache + step.vcache:
        cuda.htod_async(c, z)
    cuda.sync()
    caches = [(z.copy(), z.copy()) for _ in range(2)]
    s = cuda.stream()
    tokens = [5, 311, 17, 642]
    got = []
    for pos, tok in zip(positions, tokens):
        step.run(tok, pos, s)
        cuda.sync_stream(s)
        got.append(cuda.download(step.logits, (S.vocab,), np.float32))
        want = _oracle_step(S, W, moe, caches, tok, pos)
        assert rel_l2(got[-1], want) <= 1e-3, (pos, rel_l2(got[-1], want))
    # the last step recorded once and replayed after the first three
    # positions are rebuilt: the same logits, bit for bit
    g = step.capture(tokens[-1], positions[-1], s)
    try:
        for pos, tok in zip(positions[:-1], tokens[:-1]):
            step.run(tok, pos, s)
        for _ in range(2):
            g.launch(s)
            cuda.sync_stream(s)
            assert np.array_equal(cuda.download(step.logits, (S.vocab,), np.float32), got[-1])
    finally:
        g.close()
    assert cuda.step_errors() == 0
    cuda.destroy_stream(s)
    step.free()
    for p in allocs:
        cuda.free_device(p)
    for L in moe:
        L.free()


@pytest.mark.parametrize("fused", [True, False])
def test_decode_step_bench_shape(cuda, fused):
    # one layer at the shape the bench's decode step runs (Qwen3-30B-A3B:
    # hidden 2048, 32 query and 4 KV heads of 128, fp16 cache; the config-2
    # MoE layer, E128 / top-8 / I768 / g32), at positions 0, 1 and 1023 (the
    # bench's: 16 splits merged by the fused attention), against the oracle's
    # composition of decode.rs:263-363
    S = StepShape(hidden=2048, heads=32, kv_heads=4, head_dim=128, vocab=1024, max_seq=2048)
    step, W, moe, allocs = _build(cuda, S, NL=1, seed=47, fused=fused,
                                  moe_shape=dict(I=768, E=128, k=8, group=32, router_std=0.02))
    assert step.fused == fused
    kd = S.kv_heads * S.head_dim
    z = np.zeros(kd * S.max_seq, np.uint16)
    for c in step.kcache + step.vcache:
        cuda.htod_async(c, z)
    cuda.sync()
    caches = [(z.copy(), z.copy())]
    s = cuda.stream()
    for pos, tok in zip((0, 1, 1023), (3, 1000, 77)):
        print(f"step bench shape fused={fused} pos={pos}", flush=True)
        step.run(tok, pos, s)
        cuda.sync_stream(s)
        got = cuda.download(step.logits, (S.vocab,), np.float32)
        want = _oracle_step(S, W, moe, caches, tok, pos)
        assert rel_l2(got, want) <= 1e-3, (pos, rel_l2(got, want))
    assert cuda.step_errors() == 0
    cuda.destroy_stream(s)
    step.free()
    for p in allocs:
        cuda.free_device(p)
    for L in moe:
        L.free()


def test_capture_misuse_is_refused(cuda):
    # ending a capture that was never begun, and a stack capture inside a
    # general one, fail cleanly (no graph, the context usable after)
    s = cuda.stream()
    with pytest.raises(lp.LpError):
        cuda.capture_end(s)
    L = DeviceLayer(cuda, H=128, I=64, E=8, k=2, group=32, seed=3)
    st = lp.MoeStack(cuda, [L.desc])
    ws = cuda.alloc_device(st.ws_bytes(1))
    h = cuda.upload(np.zeros(128, np.float32))
    cuda.capture_begin(s)
    with pytest.raises(lp.LpError):
        st.capture(h, 1, ws, s)
    g = cuda.capture_end(s)  # an empty graph
    g.close()
    st.forward(h, 1, ws, s)
    cuda.sync_stream(s)
    for p in (ws, h):
        cuda.free_device(p)
    L.free()
    cuda.destroy_stream(s)


# ---- the fused launches on their own ----------------------------------------

def _rnd(rng, n, scale=1.0):
    return (scale * rng.standard_normal(n)).astype(np.float32)


@pytest.fixture(scope="module")
def K(cuda):
    return lp.Kernels(cuda)


@pytest.mark.parametrize("cols,rows,norm", [
    (2048, (4096, 512, 512), True),  # Qwen3-30B-A3B q / k / v
    (2048, (1000,), True),            # an lm_head slice
    (256, (512, 128, 128), True),     # the step test's shape (half of a 512-column chunk)
    (4096, (37,), False),             # 4096 columns, rows not a multiple of 8
    (1000, (9, 3), True),             # columns a multiple of 8 only
])
def test_rmsnorm_gemv(cuda, K, cols, rows, norm):
    rng = np.random.default_rng(cols + len(rows))
    x = _rnd(rng, cols)
    ln = (1.0 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    ws = [lp.synth_bf16(r * cols, 0.05, 3, i) for i, r in enumerate(rows)]
    dx, dln = cuda.upload(x), cuda.upload(ln)
    dw = [cuda.upload(w) for w in ws]
    dy = [cuda.alloc_device(4 * r) for r in rows]
    K.rmsnorm_gemv(dx, dln if norm else 0, 1e-6, cols, [(w, r, y) for w, r, y in zip(dw, rows, dy)])
    xn = O.rmsnorm(x, ln, 1, cols, 1e-6) if norm else x
    for w, r, y in zip(ws, rows, dy):
        assert worst_rel(cuda.download(y, (r,), np.float32), O.bf16_gemv(w, xn, r, cols)) <= 1e-4
    for p in [dx, dln, *dw, *dy]:
        cuda.free_device(p)


@pytest.mark.parametrize("rows,cols", [(2048, 4096), (256, 512), (100, 64)])
def test_gemv_add_rmsnorm(cuda, K, rows, cols):
    # two calls in a row on one stream: the arrival counter resets itself
    rng = np.random.default_rng(rows)
    w = lp.synth_bf16(rows * cols, 0.05, 5, 1)
    ln = (1.0 + 0.1 * rng.standard_normal(rows)).astype(np.float32)
    dw, dln, dhn = cuda.upload(w), cuda.upload(ln), cuda.alloc_device(4 * rows)
    for it in range(2):
        x, h = _rnd(rng, cols), _rnd(rng, rows)
        dx, dh = cuda.upload(x), cuda.upload(h)
        K.gemv_add_rmsnorm(dw, dx, rows, cols, dh, dln, 1e-6, dhn)
        want_h = O.add(h, O.bf16_gemv(w, x, rows, cols))
        assert worst_rel(cuda.download(dh, (rows,), np.float32), want_h) <= 1e-4, it
        assert worst_rel(cuda.download(dhn, (rows,), np.float32), O.rmsnorm(want_h, ln, 1, rows, 1e-6)) <= 1e-4, it
        cuda.free_device(dx)
        cuda.free_device(dh)
    for p in (dw, dln, dhn):
        cuda.free_device(p)


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("heads,kvh,pos,ms,norms", [
    (32, 4, 1023, 4096, True),   # Qwen3-30B-A3B at the bench's position: 16 splits
    (32, 4, 4095, 4096, True),   # the last position of the cache: 22 splits of 3 chunks
    (32, 4, 0, 4096, True),      # the first token
    (64, 4, 700, 1024, True),    # 16 query heads per KV head (Qwen3-235B-A22B), 6 splits of 2 chunks
    (4, 2, 5, 16, True),         # no room for split records: one split
    (8, 8, 77, 200, False),      # one query head per KV head, no norms, one split of two chunks
    (4, 1, 64, 300, True),       # pos the first row of a second chunk
])
def test_attn_fused(cuda, K, heads, kvh, pos, ms, norms):
    hd = 128
    rng = np.random.default_rng(heads * 1000 + pos)
    q, k, v = _rnd(rng, heads * hd), _rnd(rng, kvh * hd), _rnd(rng, kvh * hd)
    qn = (1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    # rows before pos hold earlier tokens, rows after it stale values
    kc, vc = _f16(_rnd(rng, kvh * ms * hd)), _f16(_rnd(rng, kvh * ms * hd))
    dq, dk, dv, dqn, dkn = (cuda.upload(a) for a in (q, k, v, qn, kn))
    dkc, dvc = cuda.upload(kc), cuda.upload(vc)
    dout, dscr = cuda.alloc_device(4 * heads * hd), cuda.alloc_device(4 * heads * ms)
    scale = 1.0 / np.sqrt(hd)
    K.attn_fused(dq, dk, dv, dqn if norms else 0, dkn if norms else 0, 1e-6, 1e6, dkc, dvc, dout, dscr, heads, kvh,
                 hd, pos, ms, scale)
    qq = O.rmsnorm(q, qn, heads, hd, 1e-6) if norms else q
    kk = O.rmsnorm(k, kn, kvh, hd, 1e-6) if norms else k
    qq, kk = O.rope(qq, heads, hd, pos, 1e6), O.rope(kk, kvh, hd, pos, 1e6)
    wkc, wvc = O.kv_append(kk, v, kc.copy(), vc.copy(), kvh, hd, pos, ms, True)
    got_kc = cuda.download(dkc, (kvh * ms * hd,), np.uint16)
    got_vc = cuda.download(dvc, (kvh * ms * hd,), np.uint16)
    row = np.zeros((kvh, ms), bool)
    row[:, pos] = True
    row = np.repeat(row.reshape(-1), hd)
    assert np.array_equal(got_kc[~row], kc[~row]) and np.array_equal(got_vc[~row], vc[~row])
    assert np.array_equal(got_vc[row], wvc[row])  # v is appended as given
    f = lambda u: u.view(np.float16).astype(np.float64)
    assert np.max(np.abs(f(got_kc[row]) - f(wkc[row])) / np.maximum(np.abs(f(wkc[row])), 1.0)) <= 2.0 ** -10
    want = O.attn_decode(qq, wkc, wvc, heads, kvh, hd, pos + 1, ms, scale, True)
    assert worst_rel(cuda.download(dout, (heads * hd,), np.float32), want) <= 1e-3
    for p in (dq, dk, dv, dqn, dkn, dkc, dvc, dout, dscr):
        cuda.free_device(p)


@pytest.mark.parametrize("heads,kvh,pos,ms,hidden", [
    (32, 4, 1023, 4096, 2048),  # Qwen3-30B-A3B: 16 splits merged, then the o projection
    (4, 2, 5, 16, 256),          # one split per KV head: each signals on its own
    (32, 2, 200, 1024, 1000),    # 16 query heads per KV head; hidden not a multiple of 8 rows
])
def test_attn_block(cuda, K, heads, kvh, pos, ms, hidden):
    # attention then h += W_o att, hn = rmsnorm(h, post_ln) in one launch,
    # twice in a row on one stream (its counters reset themselves)
    hd = 128
    rng = np.random.default_rng(heads + pos)
    qn = (1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    ln = (1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    wo = lp.synth_bf16(hidden * heads * hd, 0.05, 7, 1)
    kc, vc = _f16(_rnd(rng, kvh * ms * hd)), _f16(_rnd(rng, kvh * ms * hd))
    dqn, dkn, dln, dwo = cuda.upload(qn), cuda.upload(kn), cuda.upload(ln), cuda.upload(wo)
    dkc, dvc = cuda.upload(kc), cuda.upload(vc)
    datt, dscr, dhn = cuda.alloc_device(4 * heads * hd), cuda.alloc_device(4 * heads * ms), cuda.alloc_device(4 * hidden)
    scale = 1.0 / np.sqrt(hd)
    s = cuda.stream()
    for it, p in enumerate((pos, pos + 1)):
        q, k, v, h = _rnd(rng, heads * hd), _rnd(rng, kvh * hd), _rnd(rng, kvh * hd), _rnd(rng, hidden)
        dq, dk, dv, dh = cuda.upload(q), cuda.upload(k), cuda.upload(v), cuda.upload(h)
        K.attn_block(dq, dk, dv, dqn, dkn, 1e-6, 1e6, dkc, dvc, datt, dscr, heads, kvh, hd, p, ms, scale, dwo, dh,
                     dln, dhn, hidden, s)
        cuda.sync_stream(s)
        qq = O.rope(O.rmsnorm(q, qn, heads, hd, 1e-6), heads, hd, p, 1e6)
        kk = O.rope(O.rmsnorm(k, kn, kvh, hd, 1e-6), kvh, hd, p, 1e6)
        kc, vc = O.kv_append(kk, v, kc, vc, kvh, hd, p, ms, True)
        att = O.attn_decode(qq, kc, vc, heads, kvh, hd, p + 1, ms, scale, True)
        got_att = cuda.download(datt, (heads * hd,), np.float32)
        assert worst_rel(got_att, att) <= 1e-3, it
        # the rest from the kernel's own attention output and caches, so the
        # bound is the o projection's and the norm's
        kc = cuda.download(dkc, (kvh * ms * hd,), np.uint16)
        vc = cuda.download(dvc, (kvh * ms * hd,), np.uint16)
        want_h = O.add(h, O.bf16_gemv(wo, got_att, hidden, heads * hd))
        assert worst_rel(cuda.download(dh, (hidden,), np.float32), want_h) <= 1e-4, it
        assert worst_rel(cuda.download(dhn, (hidden,), np.float32), O.rmsnorm(want_h, ln, 1, hidden, 1e-6)) <= 1e-4, it
        for d in (dq, dk, dv, dh):
            cuda.free_device(d)
    assert cuda.step_errors() == 0  # no wait of the o projection gave up
    cuda.destroy_stream(s)
    for d in (dqn, dkn, dln, dwo, dkc, dvc, datt, dscr, dhn):
        cuda.free_device(d)


def test_attn_block_wait_that_gives_up_is_reported(cuda):
    # a context whose bound on the o projection's wait is one poll (set from
    # the host): the long attention at pos 4095 outlasts it, the wait gives
    # up, the launch still ends, and lp_step_errors_sync reports it and clears
    # the counters; a context with the normal bound then computes correctly
    import os
    hd, heads, kvh, ms, hidden, pos = 128, 32, 4, 4096, 2048, 4095
    rng = np.random.default_rng(5)
    q, k, v, h = _rnd(rng, heads * hd), _rnd(rng, kvh * hd), _rnd(rng, kvh * hd), _rnd(rng, hidden)
    wo = lp.synth_bf16(hidden * heads * hd, 0.05, 7, 2)
    kc = _f16(_rnd(rng, kvh * ms * hd))
    scale = 1.0 / np.sqrt(hd)
    os.environ["LLMPAGER_HIP_STEP_SPIN"] = "1"
    try:
        c1 = lp.Cuda(0)
    finally:
        del os.environ["LLMPAGER_HIP_STEP_SPIN"]
    for c, given_up in ((c1, True), (cuda, False)):
        K2 = lp.Kernels(c)
        ones = c.upload(np.ones(hidden, np.float32))
        bufs = [c.upload(a) for a in (q, k, v, wo, kc, kc.copy(), h.copy())]
        dq, dk, dv, dwo, dkc, dvc, dh = bufs
        datt, dscr, dhn = c.alloc_device(4 * heads * hd), c.alloc_device(4 * heads * ms), c.alloc_device(4 * hidden)
        K2.attn_block(dq, dk, dv, 0, 0, 1e-6, 1e6, dkc, dvc, datt, dscr, heads, kvh, hd, pos, ms, scale, dwo, dh,
                      ones, dhn, hidden)
        n = c.step_errors()
        assert (n > 0) == given_up, n
        if not given_up:
            got = c.download(datt, (heads * hd,), np.float32)
            want_h = O.add(h, O.bf16_gemv(wo, got, hidden, heads * hd))
            assert worst_rel(c.download(dh, (hidden,), np.float32), want_h) <= 1e-4
        for p in (*bufs, datt, dscr, dhn, ones):
            c.free_device(p)
    c1.close()


def test_fused_launches_refuse_what_they_do_not_take(cuda, K):
    d = cuda.alloc_device(1 << 16)
    with pytest.raises(lp.LpError):   # head_dim 64
        K.attn_fused(d, d, d, 0, 0, 1e-6, 1e6, d, d, d, d, 4, 2, 64, 0, 16, 0.125)
    with pytest.raises(lp.LpError):   # 3 query heads per KV head
        K.attn_fused(d, d, d, 0, 0, 1e-6, 1e6, d, d, d, d, 6, 2, 128, 0, 16, 0.125)
    with pytest.raises(lp.LpError):   # pos past the cache
        K.attn_fused(d, d, d, 0, 0, 1e-6, 1e6, d, d, d, d, 4, 2, 128, 16, 16, 0.125)
    with pytest.raises(lp.LpError):   # more than 4096 columns
        K.rmsnorm_gemv(d, 0, 1e-6, 4104, [(d, 1, d)])
    with pytest.raises(lp.LpError):   # columns not a multiple of 8
        K.gemv_add_rmsnorm(d, d, 8, 100, d, d, 1e-6, d)
    with pytest.raises(lp.LpError):   # heads x head_dim past 4096
        K.attn_block(d, d, d, 0, 0, 1e-6, 1e6, d, d, d, d, 64, 4, 128, 0, 16, 0.125, d, d, d, d, 2048)
    cuda.free_device(d)
