"""Writes the golden fixtures of this directory from the CPU oracle
(oracle/lp_oracle.c, the restatement of decode.rs:303-342, 734-749,
kimi.rs:739-779, 1155-1186 and q4g64.cu:19-99) on seeded synthetic inputs.

The fixtures pin results across hosts and library versions: tests/
test_golden.py re-runs the oracle and the input generator on them (bit for
bit), tests/test_gpu_golden.py runs the device on them (routing bit-exact,
layer outputs within the north-star tolerance).  Expert blobs of the larger
shapes are not stored: they are regenerated from the seeds by
llmpager_amd.synth_blob(s) (the reference's xorshift generator,
bench/src/main.rs:99-120), and a SHA-256 of some of them is stored instead.

    python tests/golden/make_golden.py        (writes *.npz here)
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))                 # tests/ (_oracle)
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))  # the repository (llmpager_amd)
import llmpager_amd as lp  # noqa: E402
import _oracle as O  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def layer_case(H, I, E, k, G, T, seed, gating=0, renorm=True, scaling=1.0, min_weight=0.0,
               bias=None, shared=None, bf16_x=False):
    span = (lp.blob_bytes(H, I, G) + 4095) // 4096 * 4096
    blobs = lp.synth_blobs(E, span, H, I, G, seed, 0)
    router_w = lp.synth_bf16(E * H, 0.02, seed, 1000)
    if bf16_x:
        x = lp.synth_f32_bf16(T * H, 1.0, seed, 2).reshape(T, H)
        h = lp.synth_f32_bf16(T * H, 1.0, seed, 3).reshape(T, H)
    else:
        rng = np.random.default_rng(seed)
        x = rng.standard_normal((T, H)).astype(np.float32)
        h = rng.standard_normal((T, H)).astype(np.float32)
    desc = dict(hidden=H, inter=I, experts=E, top_k=k, group=G, gating=gating, renorm=renorm,
                routed_scaling=scaling, min_weight=min_weight, router_w=router_w,
                router_bias=bias, offsets=lp.blob_offsets(H, I, G))
    bl = [blobs[e * span: e * span + lp.blob_bytes(H, I, G)] for e in range(E)]
    sh = None
    if shared is not None:
        si, sg = shared
        sblob = lp.synth_blob(H, si, sg, seed, 0, 1 << 20)
        sh = dict(blob=sblob, inter=si, group=sg, offsets=lp.blob_offsets(H, si, sg))
    hout, logits, ids, w, cnt = O.moe_layer(desc, bl, x, h, threads=8, shared_blob=sh)
    out = dict(shape=np.array([H, I, E, k, G, T, seed, gating, int(renorm)], np.int64),
               scaling=np.float32(scaling), min_weight=np.float32(min_weight),
               x=x, h=h, logits=logits, ids=ids, wts=w, cnt=cnt, h_out=hout,
               router_sha=np.array(sha(router_w)), blob_sha=np.array([sha(bl[0]), sha(bl[E - 1])]))
    if bias is not None:
        out["bias"] = np.asarray(bias, np.float32)
    if shared is not None:
        out["shared"] = np.array(shared, np.int64)
    return out


def routing_cases():
    rng = np.random.default_rng(77)
    E, k = 64, 8
    rows = [rng.standard_normal(E).astype(np.float32) for _ in range(4)]
    tie = np.zeros(E, np.float32)
    tie[[3, 9, 10, 40]] = 1.5                          # ties: lowest id first
    rows.append(tie)
    ulp = np.full(E, 0.25, np.float32)
    ulp[5] = np.nextafter(np.float32(0.25), np.float32(1))
    ulp[60] = np.nextafter(np.float32(0.25), np.float32(-1))
    rows.append(ulp)                                   # neighbours one ulp apart
    wide = (rng.standard_normal(E) * 40).astype(np.float32)
    rows.append(wide)                                  # exp underflow for most ids
    rows.append(np.full(E, -3.0e38, np.float32))       # all equal, very negative
    L = np.stack(rows)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    soft = [O.top_k_softmax(r, k, renorm) for renorm in (False, True) for r in L]
    sig = [O.sigmoid_topk(r, bias, k, True, 2.5, 0.05) for r in L]
    pad = lambda v, dt: np.concatenate([v, np.full(k - len(v), -1, dt)]).astype(dt)
    return dict(logits=L, bias=bias,
                soft_ids=np.stack([pad(i, np.int32) for i, _ in soft]),
                soft_wts=np.stack([pad(w, np.float32) for _, w in soft]),
                sig_ids=np.stack([pad(i, np.int32) for i, _ in sig]),
                sig_wts=np.stack([pad(w, np.float32) for _, w in sig]),
                k=np.int64(k), scaling=np.float32(2.5), min_weight=np.float32(0.05))


def main():
    np.savez_compressed(os.path.join(HERE, "small_layer.npz"),
                        **layer_case(128, 64, 8, 2, 32, 4, 11))
    np.savez_compressed(os.path.join(HERE, "small_sigmoid_shared.npz"),
                        **layer_case(128, 64, 16, 4, 32, 3, 12, gating=1, renorm=True, scaling=2.5,
                                     min_weight=0.05, bias=np.linspace(-0.2, 0.2, 16).astype(np.float32),
                                     shared=(128, 32)))
    np.savez_compressed(os.path.join(HERE, "config1_token.npz"),
                        **layer_case(2048, 768, 128, 8, 32, 1, 0, bf16_x=True))
    np.savez_compressed(os.path.join(HERE, "routing_adversarial.npz"), **routing_cases())
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
