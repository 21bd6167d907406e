"""One decode step of the Qwen3 MoE model composed from the library's
launchers, in the order of the reference's Decoder::step
(crates/llmpager-run/src/decode.rs:263-363):

    h = embed[token]
    per layer:  hn = rmsnorm(h, input_ln); q, k, v = W_q hn, W_k hn, W_v hn
                q, k = rmsnorm per head (q_norm, k_norm); rope(q), rope(k)
                kv_append(k, v) at pos; a = attn_decode(q, caches, pos + 1)
                h += W_o a
                hn = rmsnorm(h, post_ln); h += MoE(hn)   (lp_moe_forward: router,
                top-k, dispatch, experts and the pick-order combine on the
                device, where the reference reads the router logits back and
                ranks them on the host, decode.rs:303-342)
    logits = W_lm rmsnorm(h, final_norm)

Every launch goes to one stream with no host synchronisation, so a step can
be recorded once (Cuda.capture_begin / capture_end) and replayed.  The
attention matrices are bf16 (the reference's default core dtype,
decode.rs:25-39 with core_q4 off) and the KV cache fp16 (its default,
decode.rs:151).

Two launch sequences compute the step: the reference's own, one launch per
kernels.rs call (fused=False), and the fused one (fused=True, the default
where the shape allows it: head_dim 128, an fp16 cache, 1, 2, 4, 8 or 16
query heads per KV head, at most 16 KV heads, hidden and heads x head_dim
at most 4096), two launches per attention block:

    rmsnorm_gemv       q, k, v = W_{q,k,v} rmsnorm(h, input_ln)
    attn_block         q / k norms, rope, kv_append, attention -> a; then
                       h += W_o a and hn = rmsnorm(h, post_ln) (attn_fused and
                       gemv_add_rmsnorm in one launch)

and rmsnorm_gemv again for the final norm and the lm_head."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class StepShape:
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    max_seq: int
    eps: float = 1e-6
    rope_theta: float = 1e6
    kv_f16: bool = True


def fusable(S: StepShape) -> bool:
    """Whether the fused launches (lp_attn_fused, lp_rmsnorm_gemv,
    lp_gemv_add_rmsnorm) take this shape."""
    g = S.heads // S.kv_heads if S.kv_heads else 0
    return (S.head_dim == 128 and S.kv_f16 and S.heads % S.kv_heads == 0 and g in (1, 2, 4, 8, 16)
            and S.kv_heads <= 16 and S.hidden % 8 == 0 and S.hidden <= 4096 and S.heads * S.head_dim <= 4096)


def check_step(S: StepShape, token: int, pos: int) -> None:
    """A step's token and position must lie inside the embedding table and
    the KV cache: the row lookup (lp_bf16_row, as kernels.rs's) and the cache
    append take them unchecked."""
    if not 0 <= token < S.vocab:
        raise ValueError(f"token {token} outside the vocabulary of {S.vocab}")
    if not 0 <= pos < S.max_seq:
        raise ValueError(f"position {pos} exceeds max_seq {S.max_seq}")


@dataclass
class AttnWeights:
    """One layer's attention block: bf16 [rows, cols] matrices, f32 norm
    vectors (device addresses)."""
    q: int        # [heads * head_dim, hidden]
    k: int        # [kv_heads * head_dim, hidden]
    v: int        # [kv_heads * head_dim, hidden]
    o: int        # [hidden, heads * head_dim]
    input_ln: int  # [hidden]
    q_norm: int    # [head_dim]
    k_norm: int    # [head_dim]
    post_ln: int   # [hidden]


class DecodeStep:
    """The step's device buffers (residual, norms, q/k/v, attention output,
    KV caches, logits) and its launches.  `moe` holds one MoeLayer per layer
    (with its workspace for one token: `ws`, `ws_bytes`)."""

    def __init__(self, cuda, shape: StepShape, attn: list[AttnWeights], moe: list, embed: int,
                 final_norm: int, lm_head: int, ws: int, ws_bytes: int, fused: bool | None = None):
        import llmpager_amd as lp
        assert len(attn) == len(moe)
        self.cuda, self.shape, self.attn, self.moe = cuda, shape, attn, moe
        self.embed, self.final_norm, self.lm_head = embed, final_norm, lm_head
        self.ws, self.ws_bytes = ws, ws_bytes
        self.K = lp.Kernels(cuda)
        S = shape
        qd, kd = S.heads * S.head_dim, S.kv_heads * S.head_dim
        can_fuse = fusable(S)
        if fused and not can_fuse:
            raise ValueError(f"the fused step does not take this shape: {S}")
        self.fused = can_fuse if fused is None else fused
        cb = (2 if S.kv_f16 else 4) * kd * S.max_seq
        self.allocs = []

        def alloc(n):
            p = cuda.alloc_device(n)
            self.allocs.append(p)
            return p
        self.h, self.hn = alloc(4 * S.hidden), alloc(4 * S.hidden)
        self.q, self.k, self.v = alloc(4 * qd), alloc(4 * kd), alloc(4 * kd)
        self.att, self.proj = alloc(4 * qd), alloc(4 * S.hidden)
        self.scratch = alloc(4 * S.heads * S.max_seq)
        self.logits = alloc(4 * S.vocab)
        self.kcache = [alloc(cb) for _ in attn]
        self.vcache = [alloc(cb) for _ in attn]

    def run(self, token: int, pos: int, stream) -> None:
        """The launches of one step (token at position pos) on stream."""
        S, K, s = self.shape, self.K, stream
        hid, qd, kd = S.hidden, S.heads * S.head_dim, S.kv_heads * S.head_dim
        check_step(S, token, pos)
        K.bf16_row(self.embed, token, hid, self.h, s)
        scale = 1.0 / float(np.sqrt(S.head_dim))
        if self.fused:
            for l, (w, layer) in enumerate(zip(self.attn, self.moe)):
                K.rmsnorm_gemv(self.h, w.input_ln, S.eps, hid, [(w.q, qd, self.q), (w.k, kd, self.k),
                                                                (w.v, kd, self.v)], s)
                K.attn_block(self.q, self.k, self.v, w.q_norm, w.k_norm, S.eps, S.rope_theta, self.kcache[l],
                             self.vcache[l], self.att, self.scratch, S.heads, S.kv_heads, S.head_dim, pos,
                             S.max_seq, scale, w.o, self.h, w.post_ln, self.hn, hid, s)
                layer.forward(self.hn, self.h, 1, self.ws, s, ws_bytes=self.ws_bytes)
            K.rmsnorm_gemv(self.h, self.final_norm, S.eps, hid, [(self.lm_head, S.vocab, self.logits)], s)
            return
        for l, (w, layer) in enumerate(zip(self.attn, self.moe)):
            K.rmsnorm(self.h, w.input_ln, self.hn, 1, hid, S.eps, s)
            K.bf16_gemv(w.q, self.hn, self.q, qd, hid, s)
            K.bf16_gemv(w.k, self.hn, self.k, kd, hid, s)
            K.bf16_gemv(w.v, self.hn, self.v, kd, hid, s)
            K.rmsnorm(self.q, w.q_norm, self.q, S.heads, S.head_dim, S.eps, s)
            K.rmsnorm(self.k, w.k_norm, self.k, S.kv_heads, S.head_dim, S.eps, s)
            K.rope(self.q, S.heads, S.head_dim, pos, S.rope_theta, s)
            K.rope(self.k, S.kv_heads, S.head_dim, pos, S.rope_theta, s)
            K.kv_append(self.k, self.v, self.kcache[l], self.vcache[l], S.kv_heads, S.head_dim, pos, S.max_seq,
                        S.kv_f16, s)
            K.attn_decode(self.q, self.kcache[l], self.vcache[l], self.att, self.scratch, S.heads, S.kv_heads,
                          S.head_dim, pos + 1, S.max_seq, scale, S.kv_f16, s)
            K.bf16_gemv(w.o, self.att, self.proj, hid, qd, s)
            K.add(self.h, self.proj, hid, s)
            K.rmsnorm(self.h, w.post_ln, self.hn, 1, hid, S.eps, s)
            layer.forward(self.hn, self.h, 1, self.ws, s, ws_bytes=self.ws_bytes)
        K.rmsnorm(self.h, self.final_norm, self.hn, 1, hid, S.eps, s)
        K.bf16_gemv(self.lm_head, self.hn, self.logits, S.vocab, hid, s)

    def capture(self, token: int, pos: int, stream):
        """run() recorded once as a graph (replays repeat this token and position)."""
        self.cuda.capture_begin(stream)
        try:
            self.run(token, pos, stream)
        except Exception:
            self.cuda.capture_end(stream).close()
            raise
        return self.cuda.capture_end(stream)

    def free(self) -> None:
        for p in self.allocs:
            self.cuda.free_device(p)
        self.allocs = []
