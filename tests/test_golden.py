"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py) re-checked on this host: the seeded input
generator reproduces the hashed weights, and the oracle reproduces every
stored output bit for bit (logits, picks, weights, the updated residual)."""
import hashlib
import os

import numpy as np
import pytest

import llmpager_amd as lp
import _oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LAYERS = ["small_layer.npz", "small_sigmoid_shared.npz", "config1_token.npz"]


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def regenerate(d):
    """The fixture's weights from its seeds: (desc, blobs, shared)."""
    H, I, E, k, G, T, seed, gating, renorm = (int(v) for v in d["shape"])
    span = (lp.blob_bytes(H, I, G) + 4095) // 4096 * 4096
    blobs = lp.synth_blobs(E, span, H, I, G, seed, 0)
    router_w = lp.synth_bf16(E * H, 0.02, seed, 1000)
    bl = [blobs[e * span: e * span + lp.blob_bytes(H, I, G)] for e in range(E)]
    desc = dict(hidden=H, inter=I, experts=E, top_k=k, group=G, gating=gating, renorm=bool(renorm),
                routed_scaling=float(d["scaling"]), min_weight=float(d["min_weight"]), router_w=router_w,
                router_bias=d["bias"] if "bias" in d.files else None, offsets=lp.blob_offsets(H, I, G))
    sh = None
    if "shared" in d.files:
        si, sg = (int(v) for v in d["shared"])
        sh = dict(blob=lp.synth_blob(H, si, sg, seed, 0, 1 << 20), inter=si, group=sg,
                  offsets=lp.blob_offsets(H, si, sg))
    assert str(d["router_sha"]) == _sha(router_w)
    assert [str(v) for v in d["blob_sha"]] == [_sha(bl[0]), _sha(bl[E - 1])]
    return desc, bl, sh


@pytest.mark.parametrize("name", LAYERS)
def test_golden_layer(name):
    d = load(name)
    desc, bl, sh = regenerate(d)
    hout, logits, ids, w, cnt = O.moe_layer(desc, bl, d["x"], d["h"], threads=8, shared_blob=sh)
    assert np.array_equal(logits.view(np.uint32), d["logits"].view(np.uint32))
    assert np.array_equal(cnt, d["cnt"]) and np.array_equal(ids, d["ids"])
    assert np.array_equal(w.view(np.uint32), d["wts"].view(np.uint32))
    assert np.array_equal(hout.view(np.uint32), d["h_out"].view(np.uint32))


def test_golden_routing():
    d = load("routing_adversarial.npz")
    k = int(d["k"])
    rows = d["logits"]
    for i, (renorm, r) in enumerate([(rn, r) for rn in (False, True) for r in rows]):
        ids, w = O.top_k_softmax(r, k, renorm)
        assert np.array_equal(ids, d["soft_ids"][i][: len(ids)]) and (d["soft_ids"][i][len(ids):] == -1).all()
        assert np.array_equal(w.view(np.uint32), d["soft_wts"][i][: len(w)].view(np.uint32))
    for i, r in enumerate(rows):
        ids, w = O.sigmoid_topk(r, d["bias"], k, True, float(d["scaling"]), float(d["min_weight"]))
        assert np.array_equal(ids, d["sig_ids"][i][: len(ids)]) and (d["sig_ids"][i][len(ids):] == -1).all()
        assert np.array_equal(w.view(np.uint32), d["sig_wts"][i][: len(w)].view(np.uint32))
    # the tie row picks the tied ids lowest first, as decode.rs:740-745's stable sort does
    assert d["soft_ids"][4][:4].tolist() == [3, 9, 10, 40]
