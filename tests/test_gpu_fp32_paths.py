"""Parity of the paths the benchmark runs with full-precision activations.

Every layer test elsewhere feeds bf16-exact activations.  A stacked decode
(decode.rs:277-343 restricted to the MoE block; the layer input is the
previous layer's residual) feeds fp32 values, so these tests use N(0, 1) fp32
activations that are not bf16-exact: the grouped kernels' int8 digit images
then carry both digits, and the prefill GEMM's bf16 images a live lo part.

  - one config-1 layer (H2048/I768/E128/top-8/g32) at T = 1, 8, 32: the
    balanced gate/up and down kernels;
  - a 4-layer in-place stack at the config-1 shape (x and h the same buffer,
    as the benchmark runs it), checked layer by layer against the oracle
    given the device's input to that layer;
  - a prefill layer (T = 256, the grouped MFMA GEMMs) with fp32 x;
  - the config-4 shape (H4096/I1536/E128/top-8/g32) at T = 1 and 8, whose
    gate/up streams K in chunks;
  - a 2-layer paged stack at the config-4 shape with 16 slots per layer.

Routing (ids, order, weights) is bit-exact given the device's logits; layer
outputs within rel-L2 1e-3 on the delta h' - h."""
import ctypes as C

import numpy as np
import pytest

import llmpager_amd as lp
import _oracle as O
from _digits import assert_digit_images
from _gpu import DeviceLayer, align, rel_l2

pytestmark = pytest.mark.gpu


def fp32_normal(n: int, seed: int) -> np.ndarray:
    """N(0, 1) float32 values (not rounded to bf16)."""
    return np.random.default_rng(seed).standard_normal(n).astype(np.float32)


def _routing_equal(g_ids, g_wts, g_cnt, ids, wts, cnt):
    assert np.array_equal(g_cnt, cnt)
    for t in range(len(cnt)):
        c = cnt[t]
        assert np.array_equal(g_ids[t, :c], ids[t, :c]), t
        assert np.array_equal(g_wts[t, :c].view(np.uint32), wts[t, :c].view(np.uint32)), t


def _layer_once(cuda, L: DeviceLayer, x: np.ndarray, h: np.ndarray, inplace: bool = False):
    """Run one layer on the device; returns (h', logits, ids, wts, cnt, xd, status), xd the
    digit images of x the grouped kernels read."""
    T, H, E, k = x.shape[0], L.H, L.E, L.k
    lay = lp.ws_layout(L.desc, T)
    ws = cuda.alloc_device(lay.total)
    dh = cuda.upload(h)
    dx = dh if inplace else cuda.upload(x)
    L.layer.forward(dx, dh, T, ws)
    dl = lambda off, shape, dt: cuda.download(ws + off, shape, dt)
    out = (cuda.download(dh, (T, H), np.float32), dl(lay.logits, (T, E), np.float32),
           dl(lay.ids, (T, k), np.int32), dl(lay.wts, (T, k), np.float32), dl(lay.cnt, (T,), np.int32),
           dl(lay.xd, (T, lp.dimage_bytes(H)), np.uint8), L.layer.status(ws, T))
    for p in {ws, dh, dx}:
        cuda.free_device(p)
    return out


@pytest.mark.parametrize("T", [1, 8, 32])
def test_layer_config1_fp32_activations(cuda, T):
    L = DeviceLayer(cuda, H=2048, I=768, E=128, k=8, group=32, seed=31)
    x = fp32_normal(T * 2048, 100 + T).reshape(T, 2048)
    h = fp32_normal(T * 2048, 200 + T).reshape(T, 2048)
    gh, glog, gids, gw, gcnt, xd, status = _layer_once(cuda, L, x, h)
    assert_digit_images(xd, x)              # both digits live
    assert status[1] == 0
    want, wlog, wids, ww, wcnt = O.moe_layer(L.oracle_desc(), L.oracle_blobs(), x, h, threads=8)
    assert np.array_equal(glog.view(np.uint32), wlog.view(np.uint32))
    _routing_equal(gids, gw, gcnt, wids, ww, wcnt)
    assert rel_l2(gh - h, want - h) <= 1e-3
    L.free()


@pytest.mark.parametrize("T", [1, 32])
def test_stack_config1_inplace(cuda, T):
    # 4 layers of distinct experts and routers, the layer input being the
    # residual itself (x == h, one buffer): each layer is checked against the
    # oracle given the device's input to it, so a routing near-tie cannot turn
    # a last-place difference upstream into a different pick here.
    layers = [DeviceLayer(cuda, H=2048, I=768, E=128, k=8, group=32, seed=41, layer=l) for l in range(4)]
    h = fp32_normal(T * 2048, 300 + T).reshape(T, 2048)
    lay = lp.ws_layout(layers[0].desc, T)
    ws = cuda.alloc_device(lay.total)
    dh = cuda.upload(h)
    cur = h.copy()
    for l, L in enumerate(layers):
        L.layer.forward(dh, dh, T, ws)
        got = cuda.download(dh, (T, 2048), np.float32)
        glog = cuda.download(ws + lay.logits, (T, 128), np.float32)
        gids = cuda.download(ws + lay.ids, (T, 8), np.int32)
        gw = cuda.download(ws + lay.wts, (T, 8), np.float32)
        gcnt = cuda.download(ws + lay.cnt, (T,), np.int32)
        assert L.layer.status(ws, T)[1] == 0
        want, wlog, wids, ww, wcnt = O.moe_layer(L.oracle_desc(), L.oracle_blobs(), cur, cur.copy(), threads=8)
        assert np.array_equal(glog.view(np.uint32), wlog.view(np.uint32)), l
        _routing_equal(gids, gw, gcnt, wids, ww, wcnt)
        assert rel_l2(got - cur, want - cur) <= 1e-3, l
        cur = got
    for p in (ws, dh):
        cuda.free_device(p)
    for L in layers:
        L.free()


def test_gemm_layer_fp32_activations(cuda):
    # 256 tokens x top-8 over 128 experts (16 pairs per expert on average):
    # the grouped MFMA GEMM path (fp16 operands) on fp32 x
    T, H, E = 256, 2048, 128
    L = DeviceLayer(cuda, H=H, I=768, E=E, k=8, group=32, seed=51)
    x = fp32_normal(T * H, 51).reshape(T, H)
    h = fp32_normal(T * H, 52).reshape(T, H)
    lay = lp.ws_layout(L.desc, T)
    assert lay.tiles != lay.actimg, "this shape must take the GEMM path"
    ws = cuda.alloc_device(lay.total)
    dx, dh = cuda.upload(x), cuda.upload(h)
    L.layer.forward(dx, dh, T, ws)
    got = cuda.download(dh, (T, H), np.float32)
    glog = cuda.download(ws + lay.logits, (T, E), np.float32)
    xexp = cuda.download(ws + lay.xexp, (T,), np.int32)
    status = L.layer.status(ws, T)
    for p in (ws, dx, dh):
        cuda.free_device(p)
    assert status[1] == 0
    m = np.abs(x).max(axis=1)
    assert np.array_equal(xexp, np.frexp(m)[1] - 15)
    want = O.moe_layer(L.oracle_desc(), L.oracle_blobs(), x, h.copy(), logits_in=glog, threads=8)[0]
    assert rel_l2(got - h, want - h) <= 1e-3
    L.free()


# BASELINE config 4's layer shape (Qwen3-235B-A22B)
P_H, P_I, P_E, P_K, P_G = 4096, 1536, 128, 8, 32


@pytest.mark.parametrize("T", [1, 8])
def test_layer_config4_shape(cuda, T):
    L = DeviceLayer(cuda, H=P_H, I=P_I, E=P_E, k=P_K, group=P_G, seed=61)
    x = fp32_normal(T * P_H, 400 + T).reshape(T, P_H)
    h = fp32_normal(T * P_H, 500 + T).reshape(T, P_H)
    gh, glog, gids, gw, gcnt, xd, status = _layer_once(cuda, L, x, h)
    assert status[1] == 0
    assert_digit_images(xd, x)
    want, wlog, wids, ww, wcnt = O.moe_layer(L.oracle_desc(), L.oracle_blobs(), x, h, threads=8)
    assert np.array_equal(glog.view(np.uint32), wlog.view(np.uint32))
    _routing_equal(gids, gw, gcnt, wids, ww, wcnt)
    assert rel_l2(gh - h, want - h) <= 1e-3
    L.free()


def test_paged_stack_config4_shape(cuda):
    # Two config-4-shape layers, 16 of 128 slots per layer: batch-1 decode in
    # the reference's order (route, request the picks, re-resolve, experts,
    # deferred release) over 6 tokens; evictions happen, and every layer's
    # output matches the oracle given the device's input to it.
    layers, slots, steps = 2, 16, 6
    blob = lp.blob_bytes(P_H, P_I, P_G)
    span = align(blob)
    n = layers * P_E * span
    pin = cuda.alloc_pinned(n)
    view = np.ctypeslib.as_array((C.c_uint8 * n).from_address(pin))
    for l in range(layers):
        lp.synth_blobs(P_E, span, P_H, P_I, P_G, 7, l, out=view[l * P_E * span:(l + 1) * P_E * span])
    cfg = lp.PagerConfig(layers=layers, experts_per_layer=P_E, slots_per_layer=slots, decay_interval=256,
                         blob_bytes=blob, span=0, host_blobs=pin, host_stride=span, copy_streams=2,
                         global_pool=0)
    pg = lp.Pager(cuda, cfg)
    s = cuda.stream()
    routers = [lp.synth_bf16(P_E * P_H, 0.02, 7, 1000 + l) for l in range(layers)]
    d_routers = [cuda.upload(r) for r in routers]
    go, uo, do = lp.blob_offsets(P_H, P_I, P_G)
    descs = [lp.LayerDesc(hidden=P_H, inter=P_I, experts=P_E, top_k=P_K, group=P_G, gating=lp.GATING_SOFTMAX,
                          renorm=1, routed_scaling=1.0, router_w=d_routers[l], slot_table=pg.slot_table(l),
                          arena_base=pg.arena, slot_span=pg.span, gate_off=go, up_off=uo, down_off=do)
             for l in range(layers)]
    moe = [lp.MoeLayer(cuda, d) for d in descs]
    lay = lp.ws_layout(descs[0], 1)
    ws = cuda.alloc_device(lay.total)
    h0 = fp32_normal(steps * P_H, 77).reshape(steps, P_H)
    dh = cuda.upload(h0)
    blob_of = lambda l, e: view[(l * P_E + e) * span:(l * P_E + e) * span + blob]
    for t in range(steps):
        ht = dh + t * P_H * 4
        for l in range(layers):
            cuda.sync_stream(s)    # the previous layer's update of ht is done
            x_in = cuda.download(ht, (1, P_H), np.float32)
            moe[l].route(ht, 1, ws, s)
            cuda.sync_stream(s)
            ids = cuda.download(ws + lay.ids, (P_K,), np.int32)
            cnt = int(cuda.download(ws + lay.cnt, (1,), np.int32)[0])
            got = pg.request(l, sorted(set(int(e) for e in ids[:cnt])), s)
            moe[l].resolve(1, ws, s)
            moe[l].experts(ht, ht, 1, ws, s)
            pg.release_after(got, s)
            cuda.sync_stream(s)
            out = cuda.download(ht, (1, P_H), np.float32)
            assert moe[l].status(ws, 1, s)[1] == 0
            desc = dict(hidden=P_H, inter=P_I, experts=P_E, top_k=P_K, group=P_G, gating=0, renorm=True,
                        routed_scaling=1.0, min_weight=0.0, router_w=routers[l], router_bias=None,
                        offsets=(go, uo, do))
            want, _, wids, _, wcnt = O.moe_layer(desc, [blob_of(l, e) for e in range(P_E)], x_in, x_in.copy(),
                                                 threads=8)
            assert np.array_equal(ids[:cnt], wids[0, :wcnt[0]]), (t, l)
            assert rel_l2(out - x_in, want - x_in) <= 1e-3, (t, l)
        pg.tick()
    m = pg.metrics()
    assert m["misses"] > slots and m["fetches"] == m["misses"]
    pg.sync()
    pg.close()
    for p in d_routers + [ws, dh]:
        cuda.free_device(p)
    cuda.destroy_stream(s)
    cuda.free_pinned(pin)


def _union_waves(cuda, moe, ws, lay, T, k, wave):
    """The routed union (the dispatch's unique list) and its waves."""
    cuda.sync()
    nu = int(cuda.download(ws + lay.meta, (1,), np.int32)[0])
    uniq = cuda.download(ws + lay.uniq, (nu,), np.int32)
    ids = cuda.download(ws + lay.ids, (T, k), np.int32)
    cnt = cuda.download(ws + lay.cnt, (T,), np.int32)
    want = sorted(set(int(e) for t in range(T) for e in ids[t, :cnt[t]]))
    assert uniq.tolist() == want        # decode.rs:483-485: sorted, deduplicated
    return uniq, [(u0, min(wave, nu - u0)) for u0 in range(0, nu, wave)]


def test_paged_waves_config4_shape(cuda):
    # Config 4's shape at 32 tokens with 64 slots per layer: the ~98 experts of
    # the union do not fit, so the step runs in waves of 64 as decode.rs:489-531
    # does (request the wave, re-resolve, compute the wave's experts, add each
    # token's picks inside the wave into h once, release), against the oracle
    # with the same waves.
    T, slots, wave = 32, 64, 64
    blob = lp.blob_bytes(P_H, P_I, P_G)
    span = align(blob)
    n = P_E * span
    pin = cuda.alloc_pinned(n)
    view = np.ctypeslib.as_array((C.c_uint8 * n).from_address(pin))
    lp.synth_blobs(P_E, span, P_H, P_I, P_G, 8, 0, out=view)
    cfg = lp.PagerConfig(layers=1, experts_per_layer=P_E, slots_per_layer=slots, decay_interval=256,
                         blob_bytes=blob, span=0, host_blobs=pin, host_stride=span, copy_streams=2, global_pool=0)
    pg = lp.Pager(cuda, cfg)
    s = cuda.stream()
    router = lp.synth_bf16(P_E * P_H, 0.02, 8, 1000)
    d_router = cuda.upload(router)
    go, uo, do = lp.blob_offsets(P_H, P_I, P_G)
    desc = lp.LayerDesc(hidden=P_H, inter=P_I, experts=P_E, top_k=P_K, group=P_G, gating=lp.GATING_SOFTMAX,
                        renorm=1, routed_scaling=1.0, router_w=d_router, slot_table=pg.slot_table(0),
                        arena_base=pg.arena, slot_span=pg.span, gate_off=go, up_off=uo, down_off=do)
    moe = lp.MoeLayer(cuda, desc)
    lay = lp.ws_layout(desc, T)
    ws = cuda.alloc_device(lay.total)
    x = fp32_normal(T * P_H, 801).reshape(T, P_H)
    h = fp32_normal(T * P_H, 802).reshape(T, P_H)
    dx, dh = cuda.upload(x), cuda.upload(h)
    moe.route(dx, T, ws, s)
    uniq, waves = _union_waves(cuda, moe, ws, lay, T, P_K, wave)
    assert len(waves) == 2 and len(uniq) > slots
    glog = cuda.download(ws + lay.logits, (T, P_E), np.float32)
    with pytest.raises(lp.LpError):
        moe.experts_wave(dh, dh, T, ws, 0, 4, False, s)         # x aliasing h is refused
    for i, (u0, nw) in enumerate(waves):
        got = pg.request(0, uniq[u0:u0 + nw].tolist(), s)
        moe.resolve(T, ws, s)
        moe.experts_wave(dx, dh, T, ws, u0, nw, i == len(waves) - 1, s)
        pg.release_after(got, s)
    cuda.sync_stream(s)
    out = cuda.download(dh, (T, P_H), np.float32)
    assert moe.status(ws, T, s)[1] == 0
    odesc = dict(hidden=P_H, inter=P_I, experts=P_E, top_k=P_K, group=P_G, gating=0, renorm=True,
                 routed_scaling=1.0, min_weight=0.0, router_w=router, router_bias=None, offsets=(go, uo, do))
    blobs = [view[e * span:e * span + blob] for e in range(P_E)]
    want = O.moe_layer(odesc, blobs, x, h.copy(), logits_in=glog, wave=wave, threads=8)[0]
    assert rel_l2(out - h, want - h) <= 1e-3
    m = pg.metrics()
    assert m["misses"] == len(uniq)
    pg.sync()
    pg.close()
    for p in (d_router, ws, dx, dh):
        cuda.free_device(p)
    cuda.destroy_stream(s)
    cuda.free_pinned(pin)


@pytest.mark.parametrize("T,wave", [(5, 3), (16, 2)])
def test_waves_with_shared_mlp(cuda, T, wave):
    # every expert resident; the union computed wave by wave, the shared MLP
    # added with the last wave (kimi.rs:779), against the oracle's waves; a
    # token with no pick in a wave is left untouched by it
    L = DeviceLayer(cuda, H=128, I=64, E=8, k=2, group=32, seed=14, router_std=0.2, shared=(128, 64))
    lay = lp.ws_layout(L.desc, T)
    ws = cuda.alloc_device(lay.total)
    x = fp32_normal(T * 128, 900 + T).reshape(T, 128)
    h = fp32_normal(T * 128, 901 + T).reshape(T, 128)
    dx, dh = cuda.upload(x), cuda.upload(h)
    L.layer.route(dx, T, ws)
    uniq, waves = _union_waves(cuda, L.layer, ws, lay, T, 2, wave)
    assert len(waves) >= 2
    glog = cuda.download(ws + lay.logits, (T, 8), np.float32)
    ids = cuda.download(ws + lay.ids, (T, 2), np.int32)
    for i, (u0, nw) in enumerate(waves):
        before = cuda.download(dh, (T, 128), np.float32)
        L.layer.experts_wave(dx, dh, T, ws, u0, nw, i == len(waves) - 1)
        after = cuda.download(dh, (T, 128), np.float32)
        if i < len(waves) - 1:
            idle = [t for t in range(T) if not set(ids[t].tolist()) & set(uniq[u0:u0 + nw].tolist())]
            for t in idle:
                assert np.array_equal(before[t].view(np.uint32), after[t].view(np.uint32)), t
    out = cuda.download(dh, (T, 128), np.float32)
    assert L.layer.status(ws, T)[1] == 0
    want = O.moe_layer(L.oracle_desc(), L.oracle_blobs(), x, h.copy(), logits_in=glog, wave=wave, threads=8,
                       shared_blob=L.shared)[0]
    assert rel_l2(out - h, want - h) <= 1e-3
    for p in (ws, dx, dh):
        cuda.free_device(p)
    L.free()
