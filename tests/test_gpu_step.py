"""A whole decode step (llmpager_amd.step: per layer the attention block's
1:1 kernels and the fused MoE layer, then the final norm and the lm_head)
against the oracle's composition of the same functions in the order of
decode.rs:263-363, over several positions; and the step recorded once with
lp_graph_capture_begin / lp_graph_capture_end, whose replay equals the eager
step bit for bit.

Tolerance: the logits within rel-L2 1e-3 of the oracle's (the MoE layers'
own bound; the attention kernels are held to 1e-3 worst-relative on their
own, the rest to 1e-4)."""
import numpy as np
import pytest

import llmpager_amd as lp
import _oracle as O
from _gpu import DeviceLayer, rel_l2
from llmpager_amd.step import AttnWeights, DecodeStep, StepShape

pytestmark = pytest.mark.gpu


def _build(cuda, S: StepShape, NL: int, seed: int):
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
        moe.append(DeviceLayer(cuda, H=H, I=64, E=8, k=2, group=32, seed=seed + l, layer=l, router_std=0.1))
    embed = lp.synth_bf16(S.vocab * H, 1.0, seed, 900)
    lm = lp.synth_bf16(S.vocab * H, 0.05, seed, 901)
    fn = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    ws_bytes = max(lp.ws_layout(L.desc, 1).total for L in moe)
    ws = cuda.alloc_device(ws_bytes)
    allocs.append(ws)
    step = DecodeStep(cuda, S, attn, [L.layer for L in moe], up(embed), up(fn), up(lm), ws, ws_bytes)
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


def test_decode_step_against_oracle_and_graph(cuda):
    S = StepShape(hidden=256, heads=4, kv_heads=2, head_dim=64, vocab=700, max_seq=16)
    step, W, moe, allocs = _build(cuda, S, NL=2, seed=31)
    kd = S.kv_heads * S.head_dim
    z = np.zeros(kd * S.max_seq, np.uint16)
    for c in step.kcache + step.vcache:
        cuda.htod_async(c, z)
    cuda.sync()
    caches = [(z.copy(), z.copy()) for _ in range(2)]
    s = cuda.stream()
    tokens = [5, 311, 17, 642]
    got = []
    for pos, tok in enumerate(tokens):
        step.run(tok, pos, s)
        cuda.sync_stream(s)
        got.append(cuda.download(step.logits, (S.vocab,), np.float32))
        want = _oracle_step(S, W, moe, caches, tok, pos)
        assert rel_l2(got[-1], want) <= 1e-3, (pos, rel_l2(got[-1], want))
    # the last step recorded once and replayed after the first three
    # positions are rebuilt: the same logits, bit for bit
    g = step.capture(tokens[-1], len(tokens) - 1, s)
    try:
        for pos, tok in enumerate(tokens[:-1]):
            step.run(tok, pos, s)
        for _ in range(2):
            g.launch(s)
            cuda.sync_stream(s)
            assert np.array_equal(cuda.download(step.logits, (S.vocab,), np.float32), got[-1])
    finally:
        g.close()
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
