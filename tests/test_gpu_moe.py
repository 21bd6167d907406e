"""GPU parity of the fused MoE layer against the CPU oracle.

Bit-exact: router logits (canonical order) for batches of up to 64 tokens
(larger batches use the MFMA router: within 1e-5 of sum |x||w|), routing ids /
order / weights given the device's logits (decode.rs:734-749,
kimi.rs:1155-1186 with glibc expf), dispatch tables.
Tolerance: the layer output, rel-L2 <= 1e-3 on the MoE delta h' - h (the
north-star bound, measured on the delta so the residual cannot hide error)."""
import numpy as np
import pytest

import llmpager_amd as lp
import _oracle as O
from _gpu import DeviceLayer, rel_l2

pytestmark = pytest.mark.gpu


def _run_layer(cuda, L: DeviceLayer, T: int, seed: int):
    H, E, k = L.H, L.E, L.k
    x = lp.synth_f32_bf16(T * H, 1.0, seed, 1).reshape(T, H)
    h = lp.synth_f32_bf16(T * H, 1.0, seed, 2).reshape(T, H)
    lay = lp.ws_layout(L.desc, T)
    ws = cuda.alloc_device(lay.total)
    dx, dh = cuda.upload(x), cuda.upload(h)
    L.layer.forward(dx, dh, T, ws)
    got_h = cuda.download(dh, (T, H), np.float32)
    dl = lambda off, shape, dt: cuda.download(ws + off, shape, dt)
    out = dict(
        h=got_h,
        logits=dl(lay.logits, (T, E), np.float32),
        ids=dl(lay.ids, (T, k), np.int32),
        wts=dl(lay.wts, (T, k), np.float32),
        cnt=dl(lay.cnt, (T,), np.int32),
        gs=dl(lay.gs, (E + 1,), np.int32),
        perm=dl(lay.perm, (T * k,), np.int32),
        inv=dl(lay.inv, (T * k,), np.int32),
        uniq=dl(lay.uniq, (E,), np.int32),
        status=L.layer.status(ws, T),
    )
    for p in (ws, dx, dh):
        cuda.free_device(p)
    return x, h, out


def _check_layer(L: DeviceLayer, x, h, g, T, threads=8):
    E, k = L.E, L.k
    want_h, want_logits, want_ids, want_w, want_cnt = O.moe_layer(
        L.oracle_desc(), L.oracle_blobs(), x, h, threads=threads, shared_blob=L.shared)
    # logits: canonical order, identical bits
    assert np.array_equal(g["logits"].view(np.uint32), want_logits.view(np.uint32))
    # routing: ids, order, count and weights identical
    assert np.array_equal(g["cnt"], want_cnt)
    for t in range(T):
        c = want_cnt[t]
        assert np.array_equal(g["ids"][t, :c], want_ids[t, :c]), t
        assert np.array_equal(g["wts"][t, :c].view(np.uint32), want_w[t, :c].view(np.uint32)), t
    # dispatch: identical tables
    perm, gs, inv, uniq = O.moe_dispatch(want_ids, want_cnt, T, k, E)
    assert np.array_equal(g["gs"], gs)
    assert np.array_equal(g["perm"][:gs[E]], perm)
    assert np.array_equal(g["inv"], inv)
    assert g["status"] == (len(uniq), 0)
    assert np.array_equal(g["uniq"][:len(uniq)], uniq)
    # layer output: delta within rel-L2 1e-3
    assert rel_l2(g["h"] - h, want_h - h) <= 1e-3
    assert rel_l2(g["h"], want_h) <= 1e-4


@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("T", [1, 3, 16])
def test_layer_small(cuda, group, T):
    # write_test_checkpoint shape (convert/src/lib.rs:341-423): H128/I64/E8/k2
    L = DeviceLayer(cuda, H=128, I=64, E=8, k=2, group=group, seed=7, router_std=0.2)
    x, h, g = _run_layer(cuda, L, T, seed=11 + T)
    _check_layer(L, x, h, g, T)
    L.free()


@pytest.mark.parametrize("T", [1, 5, 40])
def test_layer_top16(cuda, T):
    # top-16 of 64 experts: the combine sums each token's picks in two
    # blocks of 8; T = 1 puts 16 picks in the sort-key dispatch.
    L = DeviceLayer(cuda, H=256, I=64, E=64, k=16, group=32, seed=9, router_std=0.2)
    x, h, g = _run_layer(cuda, L, T, seed=50 + T)
    _check_layer(L, x, h, g, T)
    L.free()


def test_layer_sigmoid_dropped_picks(cuda):
    # sigmoid gating with a min_weight that drops some of each token's
    # picks (count < k), top-12: the combine's pick count cuts its second
    # block of 8 short.
    E, k = 32, 12
    L = DeviceLayer(cuda, H=256, I=64, E=E, k=k, group=32, seed=10, router_std=0.2,
                    gating=lp.GATING_SIGMOID, renorm=False, routed_scaling=1.0, min_weight=0.7,
                    bias=np.zeros(E, np.float32))
    x, h, g = _run_layer(cuda, L, 24, seed=77)
    assert g["cnt"].min() < k
    _check_layer(L, x, h, g, 24)
    L.free()


@pytest.mark.parametrize("T", [1, 2, 8, 9, 32, 64])
def test_layer_config1(cuda, T):
    # Qwen3-30B-A3B shape: H2048, E128, top-8, I768, q4 g32, softmax + renorm.
    # T = 8: the sort-key dispatch at its 64-pick limit; 9: two token blocks;
    # 64: the largest fused-routing batch, balanced kernels at their bound.
    L = DeviceLayer(cuda, H=2048, I=768, E=128, k=8, group=32, seed=0)
    x, h, g = _run_layer(cuda, L, T, seed=T)
    _check_layer(L, x, h, g, T)
    L.free()


def test_layer_sigmoid_gating(cuda):
    # DeepSeek/Kimi-style gating: sigmoid + bias, renorm, scaling, min_weight
    rng = np.random.default_rng(5)
    bias = (rng.standard_normal(64) * 0.05).astype(np.float32)
    L = DeviceLayer(cuda, H=2048, I=1408, E=64, k=6, group=32, seed=3,
                    gating=lp.GATING_SIGMOID, renorm=True, routed_scaling=2.5,
                    min_weight=0.41, bias=bias, router_std=0.05)
    T = 16
    x, h, g = _run_layer(cuda, L, T, seed=9)
    _check_layer(L, x, h, g, T)
    assert (g["cnt"] < 6).any()  # min_weight dropped some picks
    L.free()


@pytest.mark.parametrize("T", [1, 16])
def test_layer_shared_expert(cuda, T):
    # Config 5's MoE half (DeepSeek-V2-Lite style): 64 routed experts top-6 of
    # width 1408 plus the always-on shared MLP (2 x 1408 = 2816 wide), added
    # unweighted after the routed part (kimi.rs:739-744, 779).
    rng = np.random.default_rng(11)
    bias = (rng.standard_normal(64) * 0.05).astype(np.float32)
    L = DeviceLayer(cuda, H=2048, I=1408, E=64, k=6, group=32, seed=5, gating=lp.GATING_SIGMOID,
                    renorm=True, routed_scaling=1.0, bias=bias, router_std=0.05, shared=(2816, 32))
    x, h, g = _run_layer(cuda, L, T, seed=40 + T)
    _check_layer(L, x, h, g, T)
    L.free()


@pytest.mark.parametrize("T", [1, 16])
def test_layer_config5_as_benchmarked(cuda, T):
    # Config 5's MoE layer exactly as bench.py runs it: softmax gating without
    # renormalisation (DeepSeek-V2-Lite), 64 routed experts top-6 of width
    # 1408, the shared MLP of width 2816, g32, router N(0, 0.02), the layer
    # input being the residual itself (one buffer, as in the captured stack)
    L = DeviceLayer(cuda, H=2048, I=1408, E=64, k=6, group=32, seed=5, gating=lp.GATING_SOFTMAX,
                    renorm=False, router_std=0.02, shared=(2816, 32))
    h = lp.synth_f32_bf16(T * 2048, 1.0, 5, 2).reshape(T, 2048)
    lay = lp.ws_layout(L.desc, T)
    ws = cuda.alloc_device(lay.total)
    dh = cuda.upload(h)
    L.layer.forward(dh, dh, T, ws)
    got = cuda.download(dh, (T, 2048), np.float32)
    dl = lambda off, shape, dt: cuda.download(ws + off, shape, dt)
    glog, gids = dl(lay.logits, (T, 64), np.float32), dl(lay.ids, (T, 6), np.int32)
    gw, gcnt = dl(lay.wts, (T, 6), np.float32), dl(lay.cnt, (T,), np.int32)
    assert L.layer.status(ws, T)[1] == 0
    want, wlog, wids, ww, wcnt = O.moe_layer(L.oracle_desc(), L.oracle_blobs(), h, h.copy(), threads=8,
                                             shared_blob=L.shared)
    assert np.array_equal(glog.view(np.uint32), wlog.view(np.uint32))
    assert np.array_equal(gcnt, wcnt) and np.all(wcnt == 6)
    assert np.array_equal(gids, wids)
    assert np.array_equal(gw.view(np.uint32), ww.view(np.uint32))
    assert np.all(ww.sum(axis=1) < 1.0)   # softmax mass of the top 6 only: no renormalisation
    err = rel_l2(got - h, want - h)
    assert err <= 1e-3, err
    for p in (ws, dh):
        cuda.free_device(p)
    L.free()


def test_layer_shared_expert_g64_softmax(cuda):
    # a g64 shared MLP beside g32 routed experts, softmax gating, small shape
    L = DeviceLayer(cuda, H=128, I=64, E=8, k=2, group=32, seed=8, router_std=0.2, shared=(128, 64))
    x, h, g = _run_layer(cuda, L, 5, seed=3)
    _check_layer(L, x, h, g, 5)
    L.free()


def test_null_workspace_rejected(cuda):
    # a zero-byte allocation comes back as a null address: every entry that
    # writes the workspace refuses it before launching anything, and so it
    # does a misaligned one or one shorter than the layout
    L = DeviceLayer(cuda, H=128, I=64, E=8, k=2, group=32, seed=1)
    h0 = np.arange(128, dtype=np.float32).reshape(1, 128)
    dx = cuda.upload(h0)
    need = lp.ws_layout(L.desc, 1).total
    short = cuda.alloc_device(need - 256)
    big = 1 << 20
    for call in (lambda: L.layer.route(dx, 1, 0, ws_bytes=big), lambda: L.layer.forward(dx, dx, 1, 0, ws_bytes=big),
                 lambda: L.layer.experts(dx, dx, 1, 0, ws_bytes=big), lambda: L.layer.route(dx, 1, 64, ws_bytes=big),
                 lambda: L.layer.route(dx, 1, short), lambda: L.layer.route_logits(dx, 1, short),
                 lambda: L.layer.forward(dx, dx, 1, short), lambda: L.layer.experts(dx, dx, 1, short),
                 lambda: L.layer.resolve(1, short), lambda: L.layer.status(short, 1)):
        with pytest.raises(lp.LpError):
            call()
    cuda.sync()
    assert np.array_equal(cuda.download(dx, (1, 128), np.float32), h0)
    cuda.free_device(short)
    cuda.free_device(dx)
    L.free()


def test_layer_missing_expert_flags(cuda):
    # A routed expert with no slot raises the error flag and contributes 0.
    slots = np.arange(8, dtype=np.int32)
    slots[3] = -1
    L = DeviceLayer(cuda, H=128, I=64, E=8, k=8, group=32, seed=1, slots=slots)
    T = 2
    x, h, g = _run_layer(cuda, L, T, seed=1)
    assert g["status"][1] == 1
    L.free()


def test_layer_heavy_experts(cuda):
    # Decode-sized batch on few experts: experts hold more (token, pick) pairs
    # than one staged token group, so the grouped kernels run several groups
    # per expert.
    L = DeviceLayer(cuda, H=2048, I=768, E=16, k=2, group=32, seed=12, router_std=0.3)
    T = 48
    x, h, g = _run_layer(cuda, L, T, seed=5)
    assert np.bincount(g["ids"][:, :2].ravel(), minlength=16).max() > 8
    _check_layer(L, x, h, g, T)
    L.free()


def test_layer_missing_expert_full_shape(cuda):
    # The missing-expert path at the config-1 shape: flag raised, finite out.
    slots = np.arange(128, dtype=np.int32)
    slots[::3] = -1
    L = DeviceLayer(cuda, H=2048, I=768, E=128, k=8, group=32, seed=2, slots=slots)
    x, h, g = _run_layer(cuda, L, 4, seed=2)
    assert g["status"][1] == 1
    assert np.isfinite(g["h"]).all()
    L.free()


def _zero_expert_blob(L: DeviceLayer, blob: np.ndarray) -> np.ndarray:
    # every nibble 8 (q - 8 = 0): the expert's output is exactly zero, which
    # is what the layer gives for an expert without a slot
    z = blob.copy()
    go, uo, do = lp.blob_offsets(L.H, L.I, L.group)
    for off, rows, cols in ((go, L.I, L.H), (uo, L.I, L.H), (do, L.H, L.I)):
        sb = rows * (cols // L.group) * 2
        z[off + sb: off + sb + rows * cols // 2] = 0x88
    return z


@pytest.mark.parametrize("T", [1, 4, 32])
def test_layer_missing_expert_matches_zero_expert(cuda, T):
    # Experts without a slot contribute zero (flag raised); the rest of the
    # layer, at decode batch sizes through the one-token down + combine, the
    # one-shot and the balanced grouped kernels, matches the oracle with
    # those experts zeroed.
    slots = np.arange(128, dtype=np.int32)
    slots[::3] = -1
    L = DeviceLayer(cuda, H=2048, I=768, E=128, k=8, group=32, seed=2, slots=slots)
    x, h, g = _run_layer(cuda, L, T, seed=2)
    assert g["status"][1] == 1
    present = next(b for b in L.oracle_blobs() if b is not None)
    zero = _zero_expert_blob(L, present)
    blobs = [b if b is not None else zero for b in L.oracle_blobs()]
    want_h, _, want_ids, _, want_cnt = O.moe_layer(L.oracle_desc(), blobs, x, h, threads=8)
    assert np.array_equal(g["cnt"], want_cnt)
    assert any(slots[e] < 0 for e in want_ids[0, :want_cnt[0]]) or T > 4
    assert rel_l2(g["h"] - h, want_h - h) <= 1e-3
    L.free()


def _route_logits(cuda, L: DeviceLayer, logits: np.ndarray):
    T = logits.shape[0]
    lay = lp.ws_layout(L.desc, T)
    ws = cuda.alloc_device(lay.total)
    dlg = cuda.upload(np.ascontiguousarray(logits, np.float32))
    L.layer.route_logits(dlg, T, ws)
    ids = cuda.download(ws + lay.ids, (T, L.k), np.int32)
    wts = cuda.download(ws + lay.wts, (T, L.k), np.float32)
    cnt = cuda.download(ws + lay.cnt, (T,), np.int32)
    cuda.free_device(ws)
    cuda.free_device(dlg)
    return ids, wts, cnt


def _adversarial_logits(E: int, rng) -> np.ndarray:
    rows = []
    base = rng.standard_normal(E).astype(np.float32)
    rows.append(np.zeros(E, np.float32))                       # all equal
    rows.append(np.full(E, 3.5, np.float32))
    t = base.copy(); t[[5 % E, 9 % E, 17 % E]] = t.max() + 1.0; rows.append(t)  # exact ties at the top
    t = base.copy()                                            # neighbours one ulp apart
    top = np.float32(2.0)
    for j in range(min(10, E)):
        t[(3 + j) % E] = np.nextafter(top, np.float32(-10), dtype=np.float32) if j % 2 else top
        top = np.nextafter(top, np.float32(-10), dtype=np.float32) if j % 3 == 2 else top
    rows.append(t)
    rows.append((base * 1e4).astype(np.float32))              # large magnitude
    rows.append((base * 1e-6).astype(np.float32))             # tiny spread: probability collisions
    rows.append((base * 40).astype(np.float32))               # underflowing exponentials
    t = np.linspace(-0.5, 0.5, E).astype(np.float32)[::-1].copy(); rows.append(t)
    return np.stack(rows)


@pytest.mark.parametrize("E,k", [(128, 8), (64, 6), (8, 2), (4, 2), (300, 16)])
def test_routing_bit_exact_softmax(cuda, E, k):
    rng = np.random.default_rng(E * 31 + k)
    L = DeviceLayer(cuda, H=128, I=64, E=E, k=k, group=32, seed=2)
    rnd = (rng.standard_normal((2048, E)) * rng.choice([0.01, 1, 8, 30], (2048, 1))).astype(np.float32)
    logits = np.concatenate([_adversarial_logits(E, rng), rnd])
    for renorm in (True, False):
        L.desc.renorm = int(renorm)
        ids, wts, cnt = _route_logits(cuda, L, logits)
        for t in range(logits.shape[0]):
            wi, ww = O.top_k_softmax(logits[t], k, renorm)
            assert cnt[t] == len(wi)
            assert np.array_equal(ids[t, :cnt[t]], wi), (t, renorm)
            assert np.array_equal(wts[t, :cnt[t]].view(np.uint32), ww.view(np.uint32)), (t, renorm)
    L.free()


def _division_tie_logits() -> np.ndarray:
    """A 128-expert row whose 8th and 9th experts (ids 15 < 37, logits one ulp
    apart) have different exponentials, e_37 > e_15, that divide by z to one
    probability: softmax ranks them by id (15 first) where the exponentials
    alone would take 37.  Replays a seeded search (found at draw 3827)."""
    E = 128
    rng = np.random.default_rng(1)
    for _ in range(3828):
        v = np.full(E, -3.0, np.float32) + (rng.standard_normal(E) * 0.1).astype(np.float32)
        top = rng.choice(E, 7, replace=False)
        v[top] = (3.0 + rng.random(7)).astype(np.float32)
        rest = [i for i in range(E) if i not in top]
        a, b = sorted(rng.choice(rest, 2, replace=False))
        x = np.float32(rng.uniform(0.5, 2.5))
        v[a] = x
        v[b] = np.nextafter(x, np.float32(10), dtype=np.float32)
    m = v.max()
    e = np.array([O.expf(float(np.float32(vi - m))) for vi in v], np.float32)
    z = np.float32(-0.0)
    for ei in e:
        z = np.float32(z + ei)
    assert (a, b) == (15, 37) and e[b] > e[a] and np.float32(e[a] / z) == np.float32(e[b] / z)
    return v


def test_routing_division_tie(cuda):
    # Softmax ranks by the probabilities, not the exponentials: on this row
    # the two orders pick different 8th experts (a tie after the division).
    v = _division_tie_logits()
    wi, ww = O.top_k_softmax(v, 8, True)
    assert 15 in wi and 37 not in wi
    L = DeviceLayer(cuda, H=128, I=64, E=128, k=8, group=32, seed=2)
    logits = np.stack([v, v[::-1].copy(), v])
    ids, wts, cnt = _route_logits(cuda, L, logits)
    for t in range(3):
        wi, ww = O.top_k_softmax(logits[t], 8, True)
        assert cnt[t] == len(wi) and np.array_equal(ids[t, :cnt[t]], wi), t
        assert np.array_equal(wts[t, :cnt[t]].view(np.uint32), ww.view(np.uint32)), t
    L.free()


def test_routing_bit_exact_sigmoid(cuda):
    E, k = 64, 6
    rng = np.random.default_rng(77)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    bias[[1, 2]] = 0.0
    L = DeviceLayer(cuda, H=128, I=64, E=E, k=k, group=32, seed=2, gating=lp.GATING_SIGMOID,
                    renorm=True, routed_scaling=2.5, min_weight=0.05, bias=bias)
    logits = np.concatenate([_adversarial_logits(E, rng),
                             (rng.standard_normal((1024, E)) * 3).astype(np.float32)])
    for renorm, mw in ((True, 0.05), (False, 0.0), (True, 0.0)):
        L.desc.renorm, L.desc.min_weight = int(renorm), mw
        ids, wts, cnt = _route_logits(cuda, L, logits)
        for t in range(logits.shape[0]):
            wi, ww = O.sigmoid_topk(logits[t], bias, k, renorm, 2.5, mw)
            assert cnt[t] == len(wi)
            assert np.array_equal(ids[t, :cnt[t]], wi), t
            assert np.array_equal(wts[t, :cnt[t]].view(np.uint32), ww.view(np.uint32)), t
    L.free()


def _check_route(cuda, L: DeviceLayer, T: int, seed: int, stream=None):
    """lp_moe_route on fresh x against the oracle: logits, routing, dispatch
    tables and the expert table the grouped kernels read."""
    H, E, k = L.H, L.E, L.k
    x = lp.synth_f32_bf16(T * H, 1.0, seed, 1).reshape(T, H)
    lay = lp.ws_layout(L.desc, T)
    ws = cuda.alloc_device(lay.total)
    dx = cuda.upload(x)
    L.layer.route(dx, T, ws, stream)
    cuda.sync()
    dl = lambda off, shape, dt: cuda.download(ws + off, shape, dt)
    logits = dl(lay.logits, (T, E), np.float32)
    ids, wts, cnt = dl(lay.ids, (T, k), np.int32), dl(lay.wts, (T, k), np.float32), dl(lay.cnt, (T,), np.int32)
    gs, perm, inv = dl(lay.gs, (E + 1,), np.int32), dl(lay.perm, (T * k,), np.int32), dl(lay.inv, (T * k,), np.int32)
    maxu = min(T * k, E)
    et = dl(lay.et, (maxu * 32,), np.uint8)
    cuda.free_device(ws)
    cuda.free_device(dx)

    want_logits = np.stack([O.router_logits(L.router_w, x[t], E, H) for t in range(T)])
    if T <= 64:
        # the GEMV router keeps the oracle's summation order: bit-exact
        assert np.array_equal(logits.view(np.uint32), want_logits.view(np.uint32)), T
    else:
        # the MFMA router sums exact products in another fp32 order
        w = np.abs((L.router_w.view(np.uint16).astype(np.uint32) << 16).view(np.float32)).reshape(E, H)
        bound = 1e-5 * (np.abs(x).astype(np.float64) @ w.T.astype(np.float64)) + 1e-30
        assert np.all(np.abs(logits - want_logits) <= bound), T
    # routing and dispatch are bit-exact given the device's logits
    ref_logits = logits
    want_ids = np.full((T, k), -1, np.int32)
    want_cnt = np.zeros(T, np.int32)
    for t in range(T):
        wi, ww = O.top_k_softmax(ref_logits[t], k, True)
        want_cnt[t] = len(wi)
        want_ids[t, :len(wi)] = wi
        assert np.array_equal(ids[t, :len(wi)], wi), (T, t)
        assert np.array_equal(wts[t, :len(wi)].view(np.uint32), ww.view(np.uint32)), (T, t)
    assert np.array_equal(cnt, want_cnt)
    wperm, wgs, winv, uniq = O.moe_dispatch(want_ids, want_cnt, T, k, E)
    assert np.array_equal(gs, wgs) and np.array_equal(perm[:wgs[E]], wperm) and np.array_equal(inv, winv)
    # expert table: blob address, first position, pair count, first four tokens
    blob = et.view(np.uint64)[0::4]
    i32 = et.view(np.int32).reshape(maxu, 8)
    for u in range(maxu):
        if u < len(uniq):
            e = uniq[u]
            p0, n = wgs[e], wgs[e + 1] - wgs[e]
            assert blob[u] == L.arena + int(L.slots[e]) * L.span
            assert (i32[u, 2], i32[u, 3]) == (p0, n)
            toks = [wperm[p0 + i] // k if i < n else -1 for i in range(4)]
            assert list(i32[u, 4:8]) == toks, (T, u)
        else:
            assert i32[u, 3] == 0


def test_route_sequence(cuda):
    # One context and workspace shape after shape, on either side of the
    # one-workgroup top-k + dispatch limit (T <= 64) and on two streams.
    L = DeviceLayer(cuda, H=2048, I=768, E=128, k=8, group=32, seed=4, router_std=0.05)
    for i, T in enumerate((1, 9, 64, 3, 200, 8, 1)):
        _check_route(cuda, L, T, seed=100 + i)
    # and on a second stream (its own counter slice)
    s = cuda.stream()
    for i, T in enumerate((5, 33)):
        _check_route(cuda, L, T, seed=200 + i, stream=s)
    cuda.sync()
    cuda.destroy_stream(s)
    L.free()


@pytest.mark.parametrize("E,k,T", [(8, 2, 64), (4, 2, 1), (64, 6, 17), (128, 8, 32), (300, 16, 5),
                                   (300, 16, 64), (1024, 16, 64), (1024, 16, 7), (8, 8, 8), (4, 2, 8),
                                   (16, 4, 6)])
def test_route_one_launch_tables(cuda, E, k, T):
    # The one-launch routing's tables at its sizes (T <= 64): one token block
    # (picks from LDS) and several (picks from memory), up to 1024 picks and
    # the largest expert count; 8 experts x 64 tokens put 16 picks on each.
    # One block of at most 64 picks is placed by sort keys: every token on
    # every expert (8 x 8 x 8: runs of 8, the entry naming the first 4),
    # four picks per expert (4 x 2 x 8), and a ragged mix (16 x 4 x 6).
    # A permuted slot table, so each entry's blob shows which slot it read.
    slots = np.random.default_rng(E + k).permutation(E).astype(np.int32)
    L = DeviceLayer(cuda, H=256, I=64, E=E, k=k, group=32, seed=6, router_std=0.05, slots=slots)
    _check_route(cuda, L, T, seed=400 + T)
    L.free()


@pytest.mark.parametrize("E,k,T", [(128, 8, 300), (8, 2, 1100), (300, 16, 513)])
def test_route_multiblock(cuda, E, k, T):
    # Batches above the one-workgroup limit dispatch in blocks of 256 tokens:
    # ragged last blocks, experts whose picks span several blocks (8 experts x
    # 1100 tokens), more experts than a block has tokens (300).
    L = DeviceLayer(cuda, H=256, I=64, E=E, k=k, group=32, seed=5, router_std=0.05)
    _check_route(cuda, L, T, seed=300 + T)
    L.free()
