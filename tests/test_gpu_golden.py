"""The device against the committed golden fixtures (tests/golden/*.npz):
router logits, picks and weights bit for bit, the updated residual within
rel-L2 1e-3 on the delta h' - h."""
import numpy as np
import pytest

import llmpager_amd as lp
from _gpu import DeviceLayer, rel_l2
from test_golden import LAYERS, load

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", LAYERS)
def test_golden_layer_device(cuda, name):
    d = load(name)
    H, I, E, k, G, T, seed, gating, renorm = (int(v) for v in d["shape"])
    L = DeviceLayer(cuda, H=H, I=I, E=E, k=k, group=G, seed=seed, gating=gating, renorm=bool(renorm),
                    routed_scaling=float(d["scaling"]), min_weight=float(d["min_weight"]),
                    bias=d["bias"] if "bias" in d.files else None,
                    shared=tuple(int(v) for v in d["shared"]) if "shared" in d.files else None)
    lay = lp.ws_layout(L.desc, T)
    ws = cuda.alloc_device(lay.total)
    dx, dh = cuda.upload(np.ascontiguousarray(d["x"])), cuda.upload(np.ascontiguousarray(d["h"]))
    L.layer.forward(dx, dh, T, ws)
    got = cuda.download(dh, (T, H), np.float32)
    logits = cuda.download(ws + lay.logits, (T, E), np.float32)
    ids = cuda.download(ws + lay.ids, (T, k), np.int32)
    wts = cuda.download(ws + lay.wts, (T, k), np.float32)
    cnt = cuda.download(ws + lay.cnt, (T,), np.int32)
    assert L.layer.status(ws, T)[1] == 0
    for p in (ws, dx, dh):
        cuda.free_device(p)
    L.free()
    assert np.array_equal(logits.view(np.uint32), d["logits"].view(np.uint32))
    assert np.array_equal(cnt, d["cnt"])
    for t in range(T):
        c = int(cnt[t])
        assert np.array_equal(ids[t, :c], d["ids"][t, :c])
        assert np.array_equal(wts[t, :c].view(np.uint32), d["wts"][t, :c].view(np.uint32))
    assert rel_l2(got - d["h"], d["h_out"] - d["h"]) <= 1e-3


def test_golden_routing_device(cuda):
    d = load("routing_adversarial.npz")
    k, rows = int(d["k"]), d["logits"]
    T, E = rows.shape
    for renorm in (False, True):
        L = DeviceLayer(cuda, H=128, I=64, E=E, k=k, group=32, seed=1, renorm=renorm)
        lay = lp.ws_layout(L.desc, T)
        ws = cuda.alloc_device(lay.total)
        dl = cuda.upload(np.ascontiguousarray(rows))
        L.layer.route_logits(dl, T, ws)
        ids = cuda.download(ws + lay.ids, (T, k), np.int32)
        wts = cuda.download(ws + lay.wts, (T, k), np.float32)
        cnt = cuda.download(ws + lay.cnt, (T,), np.int32)
        for t in range(T):
            i = t + (T if renorm else 0)
            c = int(cnt[t])
            assert c == int((d["soft_ids"][i] >= 0).sum()), t
            assert np.array_equal(ids[t, :c], d["soft_ids"][i][:c]), t
            assert np.array_equal(wts[t, :c].view(np.uint32), d["soft_wts"][i][:c].view(np.uint32)), t
        for p in (ws, dl):
            cuda.free_device(p)
        L.free()
