#!/usr/bin/env python3
"""MoE-layer decode throughput on one MI355X: BASELINE.json config 2.

Workload: the Qwen3-30B-A3B MoE layer shape (hidden 2048, 128 experts, top-8
softmax with renormalisation, expert FFN 2048->768->2048, q4 group 32) stacked
to 48 layers; every one of the 48 x 128 experts is resident in a per-layer
slot arena (16.3 GB of HBM), router weights bf16 N(0, 0.02), activations bf16
N(0, 1), all synthetic (seed 0).  One step = one lockstep decode of B tokens
through all 48 layers (router GEMV, top-k, dispatch, grouped q4 gate/up +
SiLU, grouped down, pick-order combine into the residual), the layer input
being the residual itself.  B = 1, 8 and 32 are measured; the headline is
B = 32.

HBM bytes per step are algorithmic: per layer the router (524,288 B), each
*unique* routed expert's q4 weights once (2,654,208 B incl. scales; unique
counts are measured, not assumed) and per token 20,480 B of activations.

Prints one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer tok/s + HBM GB/s (% of 8 TB/s), Qwen3-30B-A3B-shape q4 decode"
H, I, E, K, G, LAYERS = 2048, 768, 128, 8, 32, 48
ROUTER_BYTES = E * H * 2
REGION_BYTES = I * (H // G) * 2 + I * H // 2        # 884,736: one q4 projection incl. scales
EXPERT_BYTES = 3 * REGION_BYTES                      # 2,654,208
ACT_BYTES = H * 2 + H * 4 * 2                      # x (bf16) + h read and write
PEAK_GBPS = 8000.0
# The grouped gate/up launch of a layer is the dominant kernel.
GATEUP_KERNELS = ("lp_moe_gateup", "lp_moe_gateup_bal", "lp_moe_gateup_bal_sh", "lp_moe_gateup_bal8", "lp_moe_gateup_bal_rs",
                  "lp_moe_gateup_bal_rs8")
# lp_moe_down_comb (one token) also folds the combine into the same launch
DOWN_KERNELS = ("lp_moe_down", "lp_moe_down_wide", "lp_moe_down_bal", "lp_moe_down_bal6", "lp_moe_down_comb",
                "lp_moe_down_comb16")
CALIB_BYTES = 256 << 20   # one plain device copy of known size: the PMC byte-counter calibration
# HBM bytes per dominant-kernel launch come from rocprofv3 --pmc runs of this
# bench (FETCH_SIZE, then WRITE_SIZE, each scaled by the factor the same
# counter reads for the calibration copy), recorded with the command that
# made them and the SHA-256 of the kernel source they measured in
# profiles/traffic.json.  A record whose source hash differs from the kernel
# source in the tree is stale: traffic is then reported as null.
TRAFFIC_RECORD = os.path.join(ROOT, "profiles", "traffic.json")
KERNEL_SOURCE = os.path.join(ROOT, "llmpager_amd", "csrc", "kernels", "lp_moe.hip")


def measured_traffic(kernel: str, batch: int):
    """(bytes per launch, record) for `kernel` at `batch` from the committed
    counter record, or (None, reason) when there is none for this source."""
    import hashlib
    try:
        rec = json.load(open(TRAFFIC_RECORD))
    except (OSError, ValueError):
        return None, "no counter record"
    sha = hashlib.sha256(open(KERNEL_SOURCE, "rb").read()).hexdigest()
    for r in rec.get("records", []):
        if r.get("kernel") == kernel and r.get("batch") == batch:
            if r.get("source_sha256") != sha:
                return None, "counter record is for another kernel source"
            f = r["fetch_kib"] * r["fetch_factor"] + r["write_kib"] * r["write_factor"]
            return int(round(f * 1024)), r
    return None, "no counter record for this kernel and batch"
KERNELS = ("lp_moe_router", "lp_moe_route_fused", "lp_moe_route_fused128", "lp_moe_topk_dispatch", "lp_moe_topk", "lp_moe_dispatch", "lp_moe_disp_count",
           "lp_moe_disp_scan", "lp_moe_disp_scatter", "lp_moe_ximage", *GATEUP_KERNELS, *DOWN_KERNELS,
           "lp_moe_combine")


def log(msg: str) -> None:
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def align(v: int, a: int = 4096) -> int:
    return (v + a - 1) // a * a


class Stack:
    """The 48-layer expert stack resident on the device."""

    def __init__(self, cuda, stream, layers: int, keep_host: int):
        import llmpager_amd as lp
        self.lp, self.cuda, self.s = lp, cuda, stream
        self.span = align(lp.blob_bytes(H, I, G))
        self.offsets = lp.blob_offsets(H, I, G)
        n = E * self.span
        pin = cuda.alloc_pinned(n)
        view = np.ctypeslib.as_array((C.c_uint8 * n).from_address(pin))
        self.descs, self.allocs, self.host, self.router_host = [], [], [], []
        threads = min(16, os.cpu_count() or 1)
        for l in range(layers):
            lp.synth_blobs(E, self.span, H, I, G, 0, l, threads=threads, out=view)
            arena = cuda.alloc_device(n)
            cuda.htod_ptr_async(arena, pin, n, stream)
            rw = lp.synth_bf16(E * H, 0.02, 0, 1000 + l)
            d_rw = cuda.upload(rw, stream)
            d_slots = cuda.upload(np.arange(E, dtype=np.int32), stream)
            cuda.sync_stream(stream)
            if l < keep_host:
                self.host.append(view.copy())
                self.router_host.append(rw)
            go, uo, do = self.offsets
            self.descs.append(lp.LayerDesc(
                hidden=H, inter=I, experts=E, top_k=K, group=G, gating=lp.GATING_SOFTMAX,
                renorm=1, routed_scaling=1.0, min_weight=0.0, router_w=d_rw, router_bias=0,
                slot_table=d_slots, arena_base=arena, slot_span=self.span,
                gate_off=go, up_off=uo, down_off=do))
            self.allocs += [arena, d_rw, d_slots]
            if l % 8 == 7:
                log(f"resident layers {l + 1}/{layers}")
        cuda.free_pinned(pin)
        self.layers = [lp.MoeLayer(cuda, d) for d in self.descs]
        self.stack = lp.MoeStack(cuda, self.descs)

    def step(self, h: int, T: int, ws: int) -> None:
        """One eager pass: the library's layer-stack driver (no host sync)."""
        self.stack.forward(h, T, ws, self.s)

    def unique_counts(self, h: int, T: int, ws: int) -> list[int]:
        out = []
        for L in self.layers:
            L.forward(h, h, T, ws, self.s)
            out.append(L.status(ws, T, self.s)[0])
        return out


def run_batch(cuda, stack: Stack, B: int, steps: int, warmup: int) -> dict:
    """Each step decodes a fresh batch of B tokens (resident in HBM): it
    copies the step's B token rows into the stack's residual buffer and
    replays the 48-layer stack captured once as a HIP graph
    (lp_moe_stack_capture).  The same steps are then run eagerly through
    lp_moe_stack_forward (its time is reported too), once more with every
    kernel bracketed by events (per-kernel times), and once with a status
    readback per layer (the measured unique-expert counts)."""
    import llmpager_amd as lp
    s = stack.s
    ws = cuda.alloc_device(stack.stack.ws_bytes(B))
    n = steps + warmup
    h0 = lp.synth_f32_bf16(n * B * H, 1.0, 0, 2)
    tok_bytes = B * H * 4
    saved = cuda.upload(h0, s)
    hbuf = cuda.alloc_device(h0.nbytes)
    hcur = cuda.alloc_device(tok_bytes)
    graph = stack.stack.capture(hcur, B, ws, s)

    def restore():
        cuda.dtod_async(hbuf, saved, h0.nbytes, s)
        cuda.sync()

    def run_graph(i):
        cuda.dtod_async(hcur, saved + i * tok_bytes, tok_bytes, s)
        graph.launch(s)

    def run(i):
        stack.step(hbuf + i * tok_bytes, B, ws)

    e0, e1 = cuda.event(), cuda.event()
    for i in range(warmup):
        run_graph(steps + i)
    cuda.sync()
    cuda.record_event(e0, s)
    for i in range(steps):
        run_graph(i)
    cuda.record_event(e1, s)
    cuda.sync()
    ms = cuda.elapsed_ms(e0, e1)
    # the same steps eagerly (host launches through lp_moe_stack_forward)
    restore()
    for i in range(warmup):
        run(steps + i)
    cuda.sync()
    cuda.record_event(e0, s)
    for i in range(steps):
        run(i)
    cuda.record_event(e1, s)
    cuda.sync()
    ms_eager = cuda.elapsed_ms(e0, e1)
    graph.close()
    # the same steps again, each kernel bracketed by events on its stream
    restore()
    cuda.profile_reset()
    cuda.profile(True)
    for i in range(steps):
        run(i)
    cuda.sync()
    prof = {k: cuda.profile_read(k) for k in KERNELS}
    cuda.profile(False)
    # and once more with a status readback per layer: the measured unique counts
    restore()
    uniq = [stack.unique_counts(hbuf + i * tok_bytes, B, ws) for i in range(steps)]
    for p in (ws, hbuf, saved, hcur):
        cuda.free_device(p)
    for e in (e0, e1):
        cuda.destroy_event(e)
    u = np.array(uniq, np.int64)                       # [steps, layers]
    step_bytes = float(np.mean(u.sum(1))) * EXPERT_BYTES + LAYERS * (ROUTER_BYTES + B * ACT_BYTES)
    sec = ms / 1e3 / steps
    # dominant kernel: grouped gate/up (two of the three projections of every
    # unique expert); its algorithmic bytes are U x 2 x 884,736 per launch
    gu_bytes = float(u.sum()) * 2 * REGION_BYTES
    dominant = max(GATEUP_KERNELS, key=lambda kn: prof[kn][1])
    dom_ms, dom_n = prof[dominant]
    dom_gbps = gu_bytes / (dom_ms / 1e3) / 1e9 if dom_ms > 0 else 0.0
    dn_ms = sum(prof[kn][0] for kn in DOWN_KERNELS)
    dn_gbps = float(u.sum()) * REGION_BYTES / (dn_ms / 1e3) / 1e9 if dn_ms > 0 else 0.0
    res = dict(
        batch=B, tok_s=B / sec, ms_per_step=sec * 1e3, ms_per_step_eager=ms_eager / steps,
        tok_s_eager=B / (ms_eager / 1e3 / steps), unique_experts_per_layer=float(u.mean()),
        bytes_per_step=step_bytes, hbm_gbps=step_bytes / sec / 1e9,
        hbm_frac=step_bytes / sec / 1e9 / PEAK_GBPS,
        dominant=dict(kernel=dominant, launches=dom_n, avg_us=dom_ms * 1e3 / max(dom_n, 1),
                      bytes_per_launch=gu_bytes / max(dom_n, 1), gbps=dom_gbps,
                      frac=dom_gbps / PEAK_GBPS),
        down_gbps=dn_gbps,
        kernels_avg_us={k: v[0] * 1e3 / max(v[1], 1) for k, v in prof.items() if v[1]},
    )
    log(f"B={B}: {res['tok_s']:.1f} tok/s (graph; eager {res['tok_s_eager']:.1f}), {res['ms_per_step']:.3f} ms/step, "
        f"{res['hbm_gbps']:.0f} GB/s step, gate/up {dom_gbps:.0f} GB/s, down {dn_gbps:.0f} GB/s, "
        f"U={res['unique_experts_per_layer']:.1f}")
    return res


PREFILL_T = 2048
DISPATCH_KERNELS = ("lp_moe_topk", "lp_moe_disp_count", "lp_moe_disp_scan", "lp_moe_disp_scatter")
PREFILL_KERNELS = ("lp_moe_router", "lp_gemm_router", *DISPATCH_KERNELS, "lp_moe_ximage", "lp_gemm_tiles",
                   "lp_gemm_gateup", "lp_gemm_down", "lp_moe_combine")
MFMA_PEAK_TFLOPS = 2500.0   # MI355X dense fp16 / bf16 MFMA


def run_prefill(cuda, s, steps: int, warmup: int) -> dict:
    """Workload config 3: a 2048-token chunk through one Qwen3-30B-A3B-shape
    layer whose router logits carry a Zipf(1.1) per-expert offset
    (v_e += -1.1 ln rank_e, rank a seeded permutation of 1..128), so expert
    loads are skewed (the top expert takes ~23% of the picks).

    The logits are the device router's own (lp_moe_route on the chunk), biased
    once on the host and kept resident; a step is lp_moe_route_logits (top-k
    + dispatch from those logits) + lp_moe_experts (fp16 activation images,
    the grouped fp16 MFMA GEMMs, combine into the residual), and the router
    GEMV's measured time over the same chunk is added to it for tok/s."""
    import llmpager_amd as lp
    T = PREFILL_T
    span = align(lp.blob_bytes(H, I, G))
    host = lp.synth_blobs(E, span, H, I, G, 0, 0, threads=min(16, os.cpu_count() or 1))
    arena = cuda.upload(host, s)
    rw = lp.synth_bf16(E * H, 0.02, 0, 1000)
    d_rw = cuda.upload(rw, s)
    d_slots = cuda.upload(np.arange(E, dtype=np.int32), s)
    go, uo, do = lp.blob_offsets(H, I, G)
    desc = lp.LayerDesc(hidden=H, inter=I, experts=E, top_k=K, group=G, gating=lp.GATING_SOFTMAX,
                        renorm=1, routed_scaling=1.0, min_weight=0.0, router_w=d_rw, router_bias=0,
                        slot_table=d_slots, arena_base=arena, slot_span=span,
                        gate_off=go, up_off=uo, down_off=do)
    layer = lp.MoeLayer(cuda, desc)
    lay = lp.ws_layout(desc, T)
    assert lay.tiles != lay.actimg, "config 3 must take the grouped-GEMM path"
    ws = cuda.alloc_device(lay.total)
    x, h = lp.synth_f32_bf16(T * H, 1.0, 0, 3), lp.synth_f32_bf16(T * H, 1.0, 0, 4)
    dx, dh = cuda.upload(x, s), cuda.upload(h, s)
    cuda.sync_stream(s)     # the host copies above may go once the uploads are done
    del host
    layer.route(dx, T, ws, s)
    logits = cuda.download(ws + lay.logits, (T, E), np.float32, s)
    rank = np.random.default_rng(0).permutation(E) + 1
    biased = np.ascontiguousarray(logits + (-1.1 * np.log(rank)).astype(np.float32), np.float32)
    dl = cuda.upload(biased, s)
    cuda.sync_stream(s)

    def step():
        layer.route_logits(dl, T, ws, s)
        layer.experts(dx, dh, T, ws, s)

    for _ in range(warmup):
        step()
    e0, e1 = cuda.event(), cuda.event()
    cuda.sync()
    cuda.record_event(e0, s)
    for _ in range(steps):
        step()
    cuda.record_event(e1, s)
    cuda.sync()
    ms = cuda.elapsed_ms(e0, e1) / steps
    cuda.profile_reset()
    cuda.profile(True)
    for _ in range(steps):
        step()
    for _ in range(steps):
        layer.route(dx, T, ws, s)     # the router GEMV over the same chunk
    cuda.sync()
    prof = {k: cuda.profile_read(k) for k in PREFILL_KERNELS}
    cuda.profile(False)
    step()
    gs = cuda.download(ws + lay.gs, (E + 1,), np.int32, s)
    uniq, err = layer.status(ws, T, s)
    for p in (ws, dx, dh, dl, arena, d_rw, d_slots):
        cuda.free_device(p)
    for e in (e0, e1):
        cuda.destroy_event(e)
    assert err == 0, f"prefill step reported error flags {err}"
    avg = {k: v[0] / max(v[1], 1) for k, v in prof.items() if v[1]}   # ms per launch
    load = np.diff(gs)
    pairs = int(gs[-1])
    router_ms = avg.get("lp_gemm_router", 0.0) + avg.get("lp_moe_router", 0.0)  # one of them runs
    step_ms = ms + router_ms
    gu_flop = 2.0 * pairs * (2 * I) * H
    dn_flop = 2.0 * pairs * H * I
    rt_flop = 2.0 * T * E * H

    def tf(flop, t_ms):
        return flop / (t_ms / 1e3) / 1e12 if t_ms > 0 else 0.0

    gu_ms, dn_ms = avg["lp_gemm_gateup"], avg["lp_gemm_down"]
    gemm_tf = tf(gu_flop + dn_flop, gu_ms + dn_ms)
    res = dict(
        tokens=T, tok_s=T / (step_ms / 1e3), ms_per_step=step_ms, route_experts_ms=ms,
        flop_per_step=gu_flop + dn_flop + rt_flop, pairs=pairs, unique_experts=uniq,
        max_expert_load=int(load.max()), top_expert_share=float(load.max() / max(pairs, 1)),
        gemm=dict(gateup_us=gu_ms * 1e3, down_us=dn_ms * 1e3,
                  gateup_tflops=tf(gu_flop, gu_ms), down_tflops=tf(dn_flop, dn_ms),
                  tflops=gemm_tf, mfma_util=gemm_tf / MFMA_PEAK_TFLOPS),
        layer_tflops=tf(gu_flop + dn_flop + rt_flop, step_ms),
        dispatch_us=sum(avg.get(kn, 0.0) for kn in DISPATCH_KERNELS) * 1e3,
        combine_us=avg.get("lp_moe_combine", 0) * 1e3,
        kernels_avg_us={k: v * 1e3 for k, v in avg.items()},
    )
    log(f"prefill T={T}: {res['tok_s']:.0f} tok/s, {step_ms:.3f} ms/layer, GEMMs "
        f"{gemm_tf:.0f} TFLOP/s ({100 * res['gemm']['mfma_util']:.1f}% of fp16 MFMA), gate/up "
        f"{gu_ms * 1e3:.1f} us, down {dn_ms * 1e3:.1f} us, dispatch {res['dispatch_us']:.1f} us, "
        f"combine {res['combine_us']:.1f} us, top expert {res['top_expert_share']:.3f} of picks")
    return res


# Workload config 4: Qwen3-235B-A22B shape with expert paging.
P_H, P_I, P_E, P_K, P_G = 4096, 1536, 128, 8, 32
P_LAYERS, P_SLOTS, P_TOKENS, P_ZIPF = 94, 64, 512, 1.1


def zipf_trace(layers: int, tokens: int, E: int, k: int, s: float = P_ZIPF, seed: int = 0) -> np.ndarray:
    """[tokens, layers, k] expert ids: per (token, layer) k distinct experts
    drawn without replacement with probability proportional to rank^-s over
    a per-layer seeded ranking of the experts, in draw order (Gumbel top-k,
    which has the sequential draws' distribution)."""
    rng = np.random.default_rng(seed)
    logw = -s * np.log(np.arange(1, E + 1, dtype=np.float64))
    out = np.empty((tokens, layers, k), np.int32)
    for l in range(layers):
        expert_of_rank = rng.permutation(E)
        keys = logw[None, :] + rng.gumbel(size=(tokens, E))
        ranks = np.argsort(-keys, axis=1, kind="stable")[:, :k]
        out[:, l, :] = expert_of_rank[ranks]
    return out


def run_paged_batch(cuda, s, host, layers: int, trace: np.ndarray, B: int, slots: int, io_threads: int,
                    stage_threads: int) -> dict:
    """Config 4 in lockstep batches of B tokens (the reference's step_multi,
    decode.rs:431-532): per layer the batch's picks (the trace's), their
    union sorted by expert id, fetched and computed in waves of `slots`
    experts (decode.rs:483-531): request the wave from the pager, re-resolve
    the expert table, lp_moe_experts_wave (each token's picks inside the
    wave added into h once), release after the stream passes.  A cold pager
    over the same pageable host pack."""
    import llmpager_amd as lp
    blob = lp.blob_bytes(P_H, P_I, P_G)
    cfg = lp.PagerConfig(layers=layers, experts_per_layer=P_E, slots_per_layer=slots, decay_interval=256,
                         blob_bytes=blob, span=0, host_blobs=host.ctypes.data, host_stride=align(blob),
                         copy_streams=1, global_pool=0, source=lp.PAGER_SRC_HOST, io_threads=io_threads,
                         ring_slots=2, stage_threads=stage_threads)
    pg = lp.Pager(cuda, cfg)
    go, uo, do = lp.blob_offsets(P_H, P_I, P_G)
    d_rw = cuda.upload(lp.synth_bf16(P_E * P_H, 0.02, 0, 1000), s)   # unused by route_logits
    descs = [lp.LayerDesc(hidden=P_H, inter=P_I, experts=P_E, top_k=P_K, group=P_G, gating=lp.GATING_SOFTMAX,
                          renorm=1, routed_scaling=1.0, min_weight=0.0, router_w=d_rw, router_bias=0,
                          slot_table=pg.slot_table(l), arena_base=pg.arena, slot_span=pg.span,
                          gate_off=go, up_off=uo, down_off=do) for l in range(layers)]
    moe = [lp.MoeLayer(cuda, d) for d in descs]
    tokens = trace.shape[0] // B * B
    steps = tokens // B
    lg = np.zeros((tokens, layers, P_E), np.float32)
    np.put_along_axis(lg, trace[:tokens].astype(np.int64), (16.0 - np.arange(P_K, dtype=np.float32))[None, None, :],
                      axis=2)
    # [step][layer][token][E]: one route_logits call per (step, layer)
    dlg = cuda.upload(np.ascontiguousarray(lg.reshape(steps, B, layers, P_E).transpose(0, 2, 1, 3)), s)
    ws = cuda.alloc_device(lp.ws_layout(descs[0], B).total)
    dx = cuda.upload(lp.synth_f32_bf16(B * P_H, 1.0, 0, 3), s)
    dh = cuda.upload(lp.synth_f32_bf16(B * P_H, 1.0, 0, 4), s)
    cuda.sync()
    unions = [[sorted(set(int(e) for e in trace[st * B:(st + 1) * B, l].ravel())) for l in range(layers)]
              for st in range(steps)]
    n_waves = 0
    t0 = time.time()
    for st in range(steps):
        for l in range(layers):
            moe[l].route_logits(dlg + ((st * layers + l) * B * P_E) * 4, B, ws, s)
            U = unions[st][l]
            for u0 in range(0, len(U), slots):
                wave = U[u0:u0 + slots]
                got = pg.request(l, wave, s)
                moe[l].resolve(B, ws, s)
                moe[l].experts_wave(dx, dh, B, ws, u0, len(wave), False, s)
                pg.release_after(got, s)
                n_waves += 1
        pg.tick()
    cuda.sync()
    pg.sync()
    sec = time.time() - t0
    m = pg.metrics()
    uq, err = moe[-1].status(ws, B, s)
    pg.close()
    for p in (dlg, ws, dx, dh, d_rw):
        cuda.free_device(p)
    assert err == 0, f"paged batch decode reported error flags {err}"
    assert uq == len(unions[-1][-1]), "the device's union differs from the trace's"
    lookups = m["hits"] + m["misses"]
    mean_union = float(np.mean([len(U) for row in unions for U in row]))
    res = dict(
        batch=B, steps=steps, tokens=tokens, tok_s=tokens / sec, seconds=sec, waves=n_waves,
        waves_per_layer=n_waves / (steps * layers), mean_union=mean_union, hits=m["hits"], misses=m["misses"],
        hit_rate=m["hits"] / max(lookups, 1), bytes_fetched=m["bytes_fetched"],
        h2d_gbps=m["bytes_fetched"] / sec / 1e9, stalls=m["stalls"],
        hbm_gbps=steps * layers * mean_union * (blob - 32) / sec / 1e9,
    )
    log(f"paged B={B} ({layers} layers, {slots} slots): {res['tok_s']:.1f} tok/s, {res['waves_per_layer']:.2f} "
        f"waves per layer (union {mean_union:.1f}), hit rate {res['hit_rate']:.4f}, H2D {res['h2d_gbps']:.1f} GB/s")
    return res


def run_paged(cuda, s, layers: int, tokens: int, slots: int, io_threads: int = 4, stage_threads: int = 4) -> dict:
    """Workload config 4: H4096 / I1536 / E128 / top-8 / g32, `layers` layers,
    `slots` VRAM expert slots per layer; every expert blob sits in pageable
    host memory (the RAM tier: layers x 128 x 10.6 MB), and misses reach VRAM
    through the pager's pinned staging ring: `io_threads` I/O workers each copy
    a blob (split over `stage_threads` threads) into one of their two
    span-sized pinned buffers and DMA it to the slot on their own stream
    (pager.rs:650-718).  A `tokens`-token routing
    trace (8 distinct experts per token and layer, Zipf(1.1) over a per-layer
    ranking) drives batch-1 decode through the reference's order per layer:
    route (from logits that rank the trace's picks first), request the picks
    from the pager (the compute stream waits on their fills), re-resolve the
    expert table, run the experts, release after the stream passes.  Reports
    tok/s, hit rate and H2D GB/s over the whole trace (cold start included)."""
    import llmpager_amd as lp
    blob = lp.blob_bytes(P_H, P_I, P_G)
    span = align(blob)
    t0 = time.time()
    n = layers * P_E * span
    host = np.empty(n, np.uint8)          # pageable: no pinned copy of the pack
    threads = min(16, os.cpu_count() or 1)
    for l in range(layers):
        lp.synth_blobs(P_E, span, P_H, P_I, P_G, 0, l, threads=threads, out=host[l * P_E * span:(l + 1) * P_E * span])
    log(f"paged: host pack {n / 1e9:.1f} GB of {layers} x {P_E} experts (pageable) in {time.time() - t0:.0f} s")
    cfg = lp.PagerConfig(layers=layers, experts_per_layer=P_E, slots_per_layer=slots, decay_interval=256,
                         blob_bytes=blob, span=0, host_blobs=host.ctypes.data, host_stride=span, copy_streams=1,
                         global_pool=0, source=lp.PAGER_SRC_HOST, io_threads=io_threads, ring_slots=2,
                         stage_threads=stage_threads)
    pg = lp.Pager(cuda, cfg)
    go, uo, do = lp.blob_offsets(P_H, P_I, P_G)
    d_rw = cuda.upload(lp.synth_bf16(P_E * P_H, 0.02, 0, 1000), s)   # unused by route_logits
    descs = [lp.LayerDesc(hidden=P_H, inter=P_I, experts=P_E, top_k=P_K, group=P_G, gating=lp.GATING_SOFTMAX,
                          renorm=1, routed_scaling=1.0, min_weight=0.0, router_w=d_rw, router_bias=0,
                          slot_table=pg.slot_table(l), arena_base=pg.arena, slot_span=pg.span,
                          gate_off=go, up_off=uo, down_off=do) for l in range(layers)]
    moe = [lp.MoeLayer(cuda, d) for d in descs]
    trace = zipf_trace(layers, tokens, P_E, P_K)
    # logits that make the trace's picks the top-k, in draw order
    lg = np.zeros((tokens, layers, P_E), np.float32)
    np.put_along_axis(lg, trace.astype(np.int64), (16.0 - np.arange(P_K, dtype=np.float32))[None, None, :], axis=2)
    dlg = cuda.upload(lg, s)
    lay = lp.ws_layout(descs[0], 1)
    ws = cuda.alloc_device(lay.total)
    dx = cuda.upload(lp.synth_f32_bf16(P_H, 1.0, 0, 3), s)
    dh = cuda.upload(lp.synth_f32_bf16(P_H, 1.0, 0, 4), s)
    cuda.sync()
    picks = [[sorted(set(int(e) for e in trace[t, l])) for l in range(layers)] for t in range(tokens)]
    t0 = time.time()
    for t in range(tokens):
        for l in range(layers):
            moe[l].route_logits(dlg + ((t * layers + l) * P_E) * 4, 1, ws, s)
            got = pg.request(l, picks[t][l], s)
            moe[l].resolve(1, ws, s)
            moe[l].experts(dx, dh, 1, ws, s)
            pg.release_after(got, s)
        pg.tick()
        if t % 128 == 127:
            log(f"paged: {t + 1}/{tokens} tokens")
    cuda.sync()
    pg.sync()
    sec = time.time() - t0
    m = pg.metrics()
    uniq, err = moe[-1].status(ws, 1, s)
    pg.close()
    for p in (dlg, ws, dx, dh, d_rw):
        cuda.free_device(p)
    assert err == 0, f"paged decode reported error flags {err}"
    # the same trace in lockstep batches of 32, each layer's union in waves
    batch = run_paged_batch(cuda, s, host, layers, trace, 32, slots, io_threads, stage_threads)
    del host
    lookups = m["hits"] + m["misses"]
    # the experts' weights and scales (the trace replaces the router GEMV)
    compute_bytes = tokens * layers * P_K * (blob - 32)
    res = dict(
        layers=layers, tokens=tokens, slots_per_layer=slots, expert_bytes=blob, source="pageable host memory",
        io_threads=io_threads, stage_threads=stage_threads, ring_buffers_per_thread=2,
        staging_bytes=io_threads * 2 * span,
        tok_s=tokens / sec, seconds=sec, hits=m["hits"], misses=m["misses"],
        hit_rate=m["hits"] / max(lookups, 1), bytes_fetched=m["bytes_fetched"],
        h2d_gbps=m["bytes_fetched"] / sec / 1e9, stalls=m["stalls"],
        fetch_latency_ms_buckets=dict(zip(("<1", "<2", "<5", "<10", "<20", "<50", ">=50"), m["latency_ms_buckets"])),
        hbm_gbps=compute_bytes / sec / 1e9,
        batch32=batch,
    )
    log(f"paged ({layers} layers, {slots} slots, {tokens} tokens): {res['tok_s']:.1f} tok/s, hit rate "
        f"{res['hit_rate']:.4f}, {res['misses']} misses, H2D {res['h2d_gbps']:.1f} GB/s")
    return res


# Workload config 5: the MoE half of a DeepSeek-V2-Lite-style layer (the MLA
# attention that precedes it in the model is outside this path).
D_H, D_I, D_E, D_K, D_G, D_SH, D_LAYERS = 2048, 1408, 64, 6, 32, 2816, 26


def run_shared(cuda, s, batches, steps: int, warmup: int) -> dict:
    """Workload config 5's MoE layer: 64 routed experts top-6 (softmax, no
    renormalisation, as DeepSeek-V2-Lite) of width 1408 plus the always-on
    shared MLP of width 2816 (2 shared experts), g32, stacked over 26 layers
    (8.4 GB of distinct weights, so the 256 MB MALL cannot serve repeats) in
    lockstep decode, each step a replayed graph of the 26 layers
    (lp_moe_stack_capture); tok/s and algorithmic GB/s at each batch."""
    import llmpager_amd as lp
    span = align(lp.blob_bytes(D_H, D_I, D_G))
    go, uo, do = lp.blob_offsets(D_H, D_I, D_G)
    sgo, suo, sdo = lp.blob_offsets(D_H, D_SH, D_G)
    threads = min(16, os.cpu_count() or 1)
    allocs, layers = [], []
    d_slots = cuda.upload(np.arange(D_E, dtype=np.int32), s)
    for l in range(D_LAYERS):
        arena = cuda.upload(lp.synth_blobs(D_E, span, D_H, D_I, D_G, 5, l, threads=threads), s)
        shared = cuda.upload(lp.synth_blob(D_H, D_SH, D_G, 5, 100 + l, 1 << 20), s)
        d_rw = cuda.upload(lp.synth_bf16(D_E * D_H, 0.02, 5, 1000 + l), s)
        cuda.sync_stream(s)
        allocs += [arena, shared, d_rw]
        desc = lp.LayerDesc(hidden=D_H, inter=D_I, experts=D_E, top_k=D_K, group=D_G, gating=lp.GATING_SOFTMAX,
                            renorm=0, routed_scaling=1.0, min_weight=0.0, router_w=d_rw, router_bias=0,
                            slot_table=d_slots, arena_base=arena, slot_span=span, gate_off=go, up_off=uo,
                            down_off=do)
        desc.shared_blob, desc.shared_inter, desc.shared_group = shared, D_SH, D_G
        desc.sh_gate_off, desc.sh_up_off, desc.sh_down_off = sgo, suo, sdo
        layers.append(lp.MoeLayer(cuda, desc))
    expert_bytes = 3 * D_I * (D_H // D_G) * 2 + 3 * D_I * D_H // 2
    shared_bytes = 3 * D_SH * (D_H // D_G) * 2 + 3 * D_SH * D_H // 2
    stack = lp.MoeStack(cuda, [L.desc for L in layers])
    out = {}
    for B in batches:
        # each step: the step's B token rows into the residual buffer, then
        # the 26 layers replayed as one captured graph (as config 2's steps)
        ws = cuda.alloc_device(stack.ws_bytes(B))
        tok_bytes = B * D_H * 4
        h0 = cuda.upload(lp.synth_f32_bf16((steps + warmup) * B * D_H, 1.0, 5, 2), s)
        hcur = cuda.alloc_device(tok_bytes)
        graph = stack.capture(hcur, B, ws, s)
        for i in range(warmup):
            cuda.dtod_async(hcur, h0 + (steps + i) * tok_bytes, tok_bytes, s)
            graph.launch(s)
        e0, e1 = cuda.event(), cuda.event()
        cuda.sync()
        cuda.record_event(e0, s)
        for i in range(steps):
            cuda.dtod_async(hcur, h0 + i * tok_bytes, tok_bytes, s)
            graph.launch(s)
        cuda.record_event(e1, s)
        cuda.sync()
        graph.close()
        cuda.free_device(hcur)
        sec = cuda.elapsed_ms(e0, e1) / 1e3 / steps
        # the measured unique routed experts of every layer of every timed
        # step (each layer's input the previous layer's output, as timed)
        hstep = cuda.alloc_device(tok_bytes)
        counts = []
        for i in range(steps):
            cuda.dtod_async(hstep, h0 + i * tok_bytes, tok_bytes, s)
            for L in layers:
                L.forward(hstep, hstep, B, ws, s)
                u_l, err = L.status(ws, B, s)
                assert err == 0, f"config-5 step reported error flags {err}"
                counts.append(u_l)
        cuda.free_device(hstep)
        u = float(np.mean(counts))                          # per layer, over layers and steps
        step_bytes = D_LAYERS * (D_E * D_H * 2 + u * expert_bytes + shared_bytes + B * D_H * 12)
        out[str(B)] = dict(batch=B, tok_s=B / sec, us_per_layer=sec / D_LAYERS * 1e6, unique_experts=u,
                           unique_experts_min=int(min(counts)), unique_experts_max=int(max(counts)),
                           hbm_gbps=step_bytes / sec / 1e9, hbm_frac=step_bytes / sec / 1e9 / PEAK_GBPS)
        log(f"config 5 B={B}: {B / sec:.1f} tok/s over {D_LAYERS} MoE layers, {sec / D_LAYERS * 1e6:.1f} us "
            f"per layer, {step_bytes / sec / 1e9:.0f} GB/s (unique routed experts {u:.1f} per layer)")
        for p in (ws, h0):
            cuda.free_device(p)
        for e in (e0, e1):
            cuda.destroy_event(e)
    for p in allocs + [d_slots]:
        cuda.free_device(p)
    return out


# Workload config 5's attention half: MLA absorbed decode over bf16 latent KV.
# Qwen3-30B-A3B's attention block and vocabulary (the whole decode step)
S_HEADS, S_KV_HEADS, S_HEAD_DIM, S_VOCAB, S_MAX_SEQ = 32, 4, 128, 151936, 4096
M_HEADS, M_QK, M_C, M_CTX = 16, 576, 512, 4096


def run_mla(cuda, s, batches, steps: int) -> dict:
    """Config 5's MLA decode: 16 heads, latent rows [kv_lora 512 | rope 64]
    in bf16 N(0, 1), context 4096, batch 1 and 16, through
    lp_mla_attn_decode_batch (scores and context on MFMA, split over
    positions, partial records merged).  Each call reads every sequence's
    latent cache once: batch x 4096 x 576 x 2 bytes, the algorithmic bytes;
    calls rotate over enough distinct caches (>= 512 MB) that the 256 MB
    MALL cannot serve repeats.  Timed with events over `steps` x rotations
    calls; the kernels' own times come from the profile events."""
    import llmpager_amd as lp
    K = lp.Kernels(cuda)
    out = {}
    row_bytes = M_QK * 2
    for B in batches:
        seq_bytes = M_CTX * row_bytes
        sets = max(2, (512 << 20) // (B * seq_bytes) + 1)
        rng = np.random.default_rng(B)
        caches = []
        for _ in range(sets):
            c = rng.standard_normal(B * M_CTX * M_QK).astype(np.float32)
            caches.append(cuda.upload(((c.view(np.uint32) + 0x8000) >> 16).astype(np.uint16), s))
        q = cuda.upload((rng.standard_normal(B * M_HEADS * M_QK) * 0.05).astype(np.float32), s)
        sl = cuda.upload(np.full(B, M_CTX, np.int32), s)
        ctx = cuda.alloc_device(B * M_HEADS * M_C * 4)
        ws = cuda.alloc_device(K.mla_batch_ws_bytes(B, M_C, M_CTX))
        scale = 1.0 / np.sqrt(192.0)

        def call(i):
            K.mla_attn_decode_batch(q, caches[i % sets], seq_bytes, sl, ctx, ws, B, M_HEADS, M_QK, M_C, M_CTX,
                                    scale, s)

        for i in range(sets):
            call(i)
        n = steps * sets
        e0, e1 = cuda.event(), cuda.event()
        cuda.sync()
        cuda.record_event(e0, s)
        for i in range(n):
            call(i)
        cuda.record_event(e1, s)
        cuda.sync()
        us = cuda.elapsed_ms(e0, e1) * 1e3 / n
        cuda.profile_reset()
        cuda.profile(True)
        for i in range(n):
            call(i)
        cuda.sync()
        split_ms, split_n = cuda.profile_read("lp_mla_split")
        comb_ms, comb_n = cuda.profile_read("lp_mla_combine")
        cuda.profile(False)
        kv_bytes = B * M_CTX * row_bytes
        split_us = split_ms * 1e3 / max(split_n, 1)
        out[str(B)] = dict(batch=B, context=M_CTX, us_per_call=us, latent_kv_bytes=kv_bytes,
                           hbm_gbps=kv_bytes / (us * 1e-6) / 1e9, hbm_frac=kv_bytes / (us * 1e-6) / 1e9 / PEAK_GBPS,
                           split_us=split_us, combine_us=comb_ms * 1e3 / max(comb_n, 1),
                           split_gbps=kv_bytes / (split_us * 1e-6) / 1e9 if split_us > 0 else 0.0,
                           split_frac=kv_bytes / (split_us * 1e-6) / 1e9 / PEAK_GBPS if split_us > 0 else 0.0)
        log(f"MLA decode B={B}, context {M_CTX}: {us:.1f} us per call, {out[str(B)]['hbm_gbps']:.0f} GB/s of latent "
            f"KV ({100 * out[str(B)]['hbm_frac']:.1f}% of 8 TB/s); split kernel {split_us:.1f} us, combine "
            f"{out[str(B)]['combine_us']:.1f} us")
        for p in caches + [q, sl, ctx, ws]:
            cuda.free_device(p)
        for e in (e0, e1):
            cuda.destroy_event(e)
    return out


def cpu_model() -> str:
    """The host CPU's model name (lscpu, else /proc/cpuinfo)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(stack: Stack, B: int, budget_s: float) -> dict:
    """The reference CPU path on the host cores, in the same run: the oracle
    (oracle/, the C restatement of the reference's arithmetic, decode.rs
    routing with glibc expf, q4 dequant-then-dot GEMVs, pick-order combine)
    over the first layers kept in host memory, scaled to the 48-layer stack.

    Two variants, as the reference's own CPU path is timed:
      ref-scalar  one thread, the reference's operation order;
      ref-omp     the same arithmetic with OpenMP over each GEMV's rows, on
                  every core this process may use (the GPU box gives each
                  GPU a share of the host: OMP_NUM_THREADS, else the
                  affinity mask).
    Each at config 1 (one layer, one token) and at config 2's headline
    batch B, until its share of about budget_s seconds is spent."""
    import llmpager_amd as lp
    path = os.path.join(ROOT, "oracle", "liblp_oracle.so")
    lib = C.CDLL(path)

    class Layer(C.Structure):
        _fields_ = [
            ("hidden", C.c_int), ("inter", C.c_int), ("experts", C.c_int), ("top_k", C.c_int),
            ("group", C.c_int), ("gating", C.c_int), ("renorm", C.c_int),
            ("routed_scaling", C.c_float), ("min_weight", C.c_float),
            ("router_w", C.c_void_p), ("router_bias", C.c_void_p), ("blobs", C.c_void_p),
            ("gate_off", C.c_uint64), ("up_off", C.c_uint64), ("down_off", C.c_uint64),
            ("shared_blob", C.c_void_p), ("shared_inter", C.c_int), ("shared_group", C.c_int),
            ("sh_gate_off", C.c_uint64), ("sh_up_off", C.c_uint64), ("sh_down_off", C.c_uint64)]

    vp = C.c_void_p
    lib.lpo_moe_layer.argtypes = [C.POINTER(Layer), vp, vp, C.c_int, vp, vp, vp, vp, vp, C.c_int,
                                  C.c_int]
    lib.lpo_moe_layer.restype = C.c_int
    try:
        share = len(os.sched_getaffinity(0))
    except AttributeError:
        share = os.cpu_count() or 1
    all_threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or share
    layers = []
    go, uo, do = stack.offsets
    for hb, rw in zip(stack.host, stack.router_host):
        ptrs = (C.c_void_p * E)(*[hb.ctypes.data + e * stack.span for e in range(E)])
        layers.append((Layer(hidden=H, inter=I, experts=E, top_k=K, group=G, gating=0, renorm=1,
                             routed_scaling=1.0, min_weight=0.0, router_w=rw.ctypes.data,
                             blobs=C.cast(ptrs, vp), gate_off=go, up_off=uo, down_off=do), ptrs))

    def leg(batch: int, threads: int, seconds: float, min_passes: int = 20) -> dict:
        # one untimed warm-up pass, then at least min_passes timed layer
        # passes (more while the time share lasts); the median pass is the
        # figure, with the spread beside it
        h = lp.synth_f32_bf16(batch * H, 1.0, 0, 2).reshape(batch, H)
        x = np.empty_like(h)

        def one(L):
            x[:] = h
            rc = lib.lpo_moe_layer(C.byref(L), x.ctypes.data, h.ctypes.data, batch, None, None, None,
                                   None, None, 0, threads)
            assert rc == 0

        one(layers[0][0])
        times, t0 = [], time.perf_counter()
        while len(times) < min_passes or time.perf_counter() - t0 < seconds:
            for L, _ in layers:
                p0 = time.perf_counter()
                one(L)
                times.append(time.perf_counter() - p0)
        dt = time.perf_counter() - t0
        med = float(np.median(times))
        per_step = med * LAYERS
        log(f"cpu baseline: batch {batch} on {threads} thread(s): {len(times)} layer passes in {dt:.1f} s, "
            f"median {med * 1e3:.2f} ms per layer (min {min(times) * 1e3:.2f}, max {max(times) * 1e3:.2f})")
        return dict(batch=batch, threads=threads, layer_passes=len(times), seconds=round(dt, 3),
                    ms_per_layer=med * 1e3, ms_per_layer_min=min(times) * 1e3, ms_per_layer_max=max(times) * 1e3,
                    tok_s=batch / per_step)

    legs = {
        "config1_scalar": leg(1, 1, budget_s * 0.1),
        "config1_omp": leg(1, all_threads, budget_s * 0.1),
        f"config2_b{B}_scalar": leg(B, 1, budget_s * 0.4),
        f"config2_b{B}_omp": leg(B, all_threads, budget_s * 0.4),
    }
    head = legs[f"config2_b{B}_omp"]
    return dict(value=head["tok_s"], unit="tok/s", cores=all_threads, kind="port",
                sample=f"oracle lpo_moe_layer (the reference's CPU semantics in C, OpenMP over GEMV rows): "
                       f"median of {head['layer_passes']} layer passes of batch {B} (after a warm-up pass) over "
                       f"the first {len(layers)} of the 48 layers, scaled to 48 layers; config-1 and "
                       f"single-thread legs in 'legs'",
                cpu_model=cpu_model(), nproc=os.cpu_count(), affinity_cpus=share,
                legs={k: _rounded(v) for k, v in legs.items()})


def _rounded(d):
    if isinstance(d, dict):
        return {k: _rounded(v) for k, v in d.items()}
    return round(d, 4) if isinstance(d, float) else d


def run_step(cuda, s, stack: "Stack", steps: int, warmup: int, pos: int = 1023, graph: bool = True) -> dict:
    """Config 2's model as one whole decode step of one token (the reference's
    Decoder::step, decode.rs:263-363, llmpager_amd.step): per layer the
    attention block (bf16 q/k/v/o for 32 query and 4 KV heads of 128, q/k
    norms, rope, the fp16 KV cache, attention over pos + 1 positions) and the
    resident MoE layer, then the final norm and the 151,936-row bf16 lm_head.
    Random-init attention and lm_head weights (N(0, 0.02) bf16; one host copy
    uploaded into every layer's own buffers, so no layer's weights are
    another's), the KV caches filled with a small constant.  The step is
    recorded once at position `pos` (lp_graph_capture_begin / end) and
    replayed; a timed step is the replay plus the logits' readback (into
    page-locked memory) and the host argmax, as the reference's greedy step
    does; the replays alone are timed too.  Per-kernel times come from one
    eager step with events.  Both launch sequences are measured: the fused
    one (three launches per attention block) and the reference's own (one
    launch per kernels.rs call).  graph=False times eager steps instead of
    replays (for profilers that do not follow graph launches)."""
    import llmpager_amd as lp
    from llmpager_amd.step import AttnWeights, DecodeStep, StepShape
    S = StepShape(hidden=H, heads=S_HEADS, kv_heads=S_KV_HEADS, head_dim=S_HEAD_DIM, vocab=S_VOCAB,
                  max_seq=S_MAX_SEQ)
    qd, kd = S.heads * S.head_dim, S.kv_heads * S.head_dim
    shapes = dict(q=qd * H, k=kd * H, v=kd * H, o=H * qd)
    host = {k: lp.synth_bf16(n, 0.02, 0, 2000 + i) for i, (k, n) in enumerate(shapes.items())}
    ones_h = np.ones(H, np.float32)
    ones_d = np.ones(S.head_dim, np.float32)
    allocs = []

    def up(a):
        p = cuda.upload(a, s)
        allocs.append(p)
        return p
    attn = [AttnWeights(q=up(host["q"]), k=up(host["k"]), v=up(host["v"]), o=up(host["o"]), input_ln=up(ones_h),
                        q_norm=up(ones_d), k_norm=up(ones_d), post_ln=up(ones_h)) for _ in range(LAYERS)]
    lm = up(lp.synth_bf16(S.vocab * H, 0.02, 0, 2100))
    fn = up(ones_h)
    ws_bytes = stack.stack.ws_bytes(1)
    ws = cuda.alloc_device(ws_bytes)
    allocs.append(ws)
    weight_bytes = LAYERS * 2 * sum(shapes.values()) + 2 * S.vocab * H
    kv_bytes = LAYERS * 2 * 2 * kd * (pos + 1)
    moe_bytes = LAYERS * (K * EXPERT_BYTES + ROUTER_BYTES + ACT_BYTES)  # one token: k distinct experts
    pinned = cuda.alloc_pinned(4 * S.vocab)
    logits = np.ctypeslib.as_array(C.cast(pinned, C.POINTER(C.c_float)), (S.vocab,))
    names = ["lp_bf16_row_to_f32", "lp_rmsnorm", "lp_bf16_gemv", "lp_rope", "lp_kv_append_f16", "lp_attn_split_f16",
             "lp_attn_combine", "lp_add", "lp_moe_route_fused", "lp_moe_route_fused128", "lp_moe_gateup_bal",
             "lp_moe_gateup_bal8", "lp_moe_down_comb", "lp_moe_down_comb16", "lp_rmsnorm_gemv_c4",
             "lp_attn_fused_g8", "lp_gemv_add_rmsnorm_c8", "lp_attn_block_g8"]

    def measure(fused: bool) -> dict:
        # the embedding gather reads one row: the lm_head's table serves as it
        step = DecodeStep(cuda, S, attn, stack.layers, lm, fn, lm, ws, ws_bytes, fused=fused)
        for c in step.kcache + step.vcache:
            cuda.memset_async(c, 0x20, 2 * kd * S.max_seq, s)  # fp16 0x2020: 0.0083
        cuda.sync_stream(s)
        # one eager step with events: per-kernel times
        step.run(7, pos, s)
        cuda.sync_stream(s)
        cuda.profile(True)
        cuda.profile_reset()
        step.run(7, pos, s)
        cuda.sync_stream(s)
        kern = {}
        for n in names:
            ms, cnt = cuda.profile_read(n)
            if cnt:
                kern[n] = {"launches": int(cnt), "us": ms * 1000.0}
        cuda.profile(False)
        moe_us = sum(v["us"] for k, v in kern.items() if k.startswith("lp_moe"))
        g = step.capture(7, pos, s) if graph else None
        one = (lambda: g.launch(s)) if graph else (lambda: step.run(7, pos, s))
        e0, e1 = cuda.event(), cuda.event()
        for _ in range(warmup):
            one()
        cuda.sync_stream(s)
        cuda.record_event(e0, s)
        for _ in range(steps):
            one()
        cuda.record_event(e1, s)
        cuda.sync_stream(s)
        graph_ms = cuda.elapsed_ms(e0, e1) / steps
        best = None
        t0 = time.perf_counter()
        for _ in range(steps):
            one()
            cuda.dtoh_ptr_async(pinned, step.logits, 4 * S.vocab, s)
            cuda.sync_stream(s)
            best = int(np.argmax(logits))
        wall_ms = (time.perf_counter() - t0) * 1000.0 / steps
        if g is not None:
            g.close()
        for e in (e0, e1):
            cuda.destroy_event(e)
        step.free()
        return {
            "fused": fused, "graph": graph, "tok_s": 1000.0 / wall_ms, "ms_per_step": wall_ms,
            "graph_ms_per_step": graph_ms, "graph_tok_s": 1000.0 / graph_ms,
            "launches_per_step": sum(v["launches"] for v in kern.values()),
            "hbm_gbps_graph": (weight_bytes + kv_bytes + moe_bytes) / (graph_ms * 1e-3) / 1e9,
            "moe_us_per_step": moe_us, "attn_and_head_us_per_step": sum(v["us"] for v in kern.values()) - moe_us,
            "kernels": kern, "argmax": best,
        }

    fused = measure(True)
    ref_seq = measure(False)
    waits_given_up = cuda.step_errors()
    if waits_given_up:
        log(f"decode step: {waits_given_up} bounded waits gave up (results invalid)")
    cuda.free_pinned(pinned)
    for p in allocs:
        cuda.free_device(p)
    out = dict(fused)
    # both launch sequences compute the same step: at full size their greedy
    # tokens must agree (the parity tests pin the logits at smaller sizes)
    out.update({"position": pos, "layers": LAYERS, "waits_given_up": waits_given_up,
                "argmax_agrees": fused["argmax"] == ref_seq["argmax"],
                "attn_weight_bytes": weight_bytes, "kv_bytes": kv_bytes,
                "moe_bytes": moe_bytes,
                "reference_launch_sequence": {k: ref_seq[k] for k in ("tok_s", "ms_per_step", "graph_ms_per_step",
                                                                      "launches_per_step", "argmax")}})
    for r in (fused, ref_seq):
        log(f"decode step B=1 at position {pos} ({'fused' if r['fused'] else 'one launch per kernels.rs call'}, "
            f"{r['launches_per_step']} launches): {r['tok_s']:.1f} tok/s ({r['ms_per_step']:.3f} ms with the logits' "
            f"readback and argmax; graph replay {r['graph_ms_per_step']:.3f} ms, {r['hbm_gbps_graph']:.0f} GB/s), "
            f"MoE {r['moe_us_per_step'] / 1000:.3f} ms + attention, norms and lm_head "
            f"{r['attn_and_head_us_per_step'] / 1000:.3f} ms of kernel time (eager step with events)")
    log(f"decode step: greedy token {fused['argmax']} (fused) and {ref_seq['argmax']} (one launch per call): "
        f"{'agree' if out['argmax_agrees'] else 'DIFFER'}")
    return out


def main() -> int:
    global LAYERS
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batches", default="1,8,32")
    ap.add_argument("--headline", type=int, default=32)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--cpu-seconds", type=float, default=24.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the config-3 prefill leg")
    ap.add_argument("--prefill-only", action="store_true")
    ap.add_argument("--no-paged", action="store_true", help="skip the config-4 paging leg")
    ap.add_argument("--no-shared", action="store_true", help="skip the config-5 shared-expert leg")
    ap.add_argument("--paged-only", action="store_true")
    ap.add_argument("--no-mla", action="store_true", help="skip the config-5 MLA attention leg")
    ap.add_argument("--mla-only", action="store_true")
    ap.add_argument("--shared-only", action="store_true")
    ap.add_argument("--no-step", action="store_true", help="skip the whole decode step leg (attention + MoE)")
    ap.add_argument("--step-only", action="store_true")
    ap.add_argument("--step-eager", action="store_true", help="time the decode step's eager launches, not a graph")
    ap.add_argument("--paged-layers", type=int, default=P_LAYERS)
    ap.add_argument("--paged-tokens", type=int, default=P_TOKENS)
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only: this build's MoE path runs on a single MI355X "
              f"(the multi-GPU expert-parallel split is a design, not built); got --gpus {a.gpus}",
              file=sys.stderr)
        return 2
    LAYERS = a.layers
    batches = [int(b) for b in a.batches.split(",")]
    if a.headline not in batches:
        batches.append(a.headline)

    import llmpager_amd as lp
    cuda = lp.Cuda(0)
    s = cuda.stream()
    # a plain device-to-device copy of CALIB_BYTES (outside every timed region):
    # under rocprofv3 --pmc it calibrates FETCH_SIZE / WRITE_SIZE per byte
    ca, cb = cuda.alloc_device(CALIB_BYTES), cuda.alloc_device(CALIB_BYTES)
    cuda.dtod_async(cb, ca, CALIB_BYTES, s)
    cuda.sync()
    cuda.free_device(ca)
    cuda.free_device(cb)
    other = a.paged_only or a.prefill_only or a.shared_only or a.step_only
    mla = None if a.no_mla or other else run_mla(cuda, s, (1, 16), a.steps)
    if a.mla_only:
        print(json.dumps({"mla": _rounded(mla)}), flush=True)
        cuda.close()
        return 0
    prefill = (None if a.no_prefill or a.paged_only or a.shared_only or a.step_only
               else run_prefill(cuda, s, a.steps, a.warmup))
    if a.prefill_only:
        print(json.dumps({"prefill": prefill}), flush=True)
        cuda.close()
        return 0
    paged = None if a.no_paged or a.shared_only or a.step_only else run_paged(cuda, s, a.paged_layers, a.paged_tokens, P_SLOTS)
    shared = None if a.no_shared or a.paged_only or a.step_only else run_shared(cuda, s, (1, 16), a.steps, a.warmup)
    if a.shared_only:
        print(json.dumps({"shared": _rounded(shared)}), flush=True)
        cuda.close()
        return 0
    if a.paged_only:
        print(json.dumps({"paged": paged}), flush=True)
        cuda.close()
        return 0
    log(f"building the {LAYERS}-layer resident stack ({LAYERS * E} experts)")
    stack = Stack(cuda, s, LAYERS, keep_host=0 if a.no_cpu or a.step_only else 2)
    dstep = None if a.no_step else run_step(cuda, s, stack, a.steps, a.warmup, graph=not a.step_eager)
    if a.step_only:
        print(json.dumps({"decode_step": _rounded(dstep)}), flush=True)
        cuda.close()
        return 0
    results = {}
    for B in batches:
        results[B] = run_batch(cuda, stack, B, a.steps, a.warmup)
    hl = results[a.headline]
    cpu = None if a.no_cpu else cpu_baseline(stack, a.headline, a.cpu_seconds)
    dom = hl["dominant"]
    traffic, trec = measured_traffic(dom["kernel"], a.headline)
    traffic_src = (f"rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE ({trec['command']}), scaled by the "
                   f"calibration copy's factors" if traffic is not None else trec)
    line = {
        "metric": METRIC,
        "value": round(hl["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(hl["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8 MFMA (q4 weights x 16-bit fixed-point activations as two int8 digits per 32 columns), fp32 accumulate",
        "data": "synthetic",
        "config": {
            "workload": f"config2: {LAYERS}-layer Qwen3-30B-A3B-shape MoE stack, lockstep decode "
                        f"batch {a.headline}, all {LAYERS * E} experts resident",
            "hidden": H, "inter": I, "experts": E, "top_k": K, "group": G, "layers": LAYERS,
            "batch": a.headline, "parallelism": "none (one GPU)",
        },
        "hbm_gbps": round(hl["hbm_gbps"], 1),
        "hbm_frac": round(hl["hbm_frac"], 4),
        "roofline": {
            "bound": "hbm",
            "kernel": dom["kernel"],
            "bytes_per_launch": round(dom["bytes_per_launch"]),
            "achieved": round(dom["gbps"], 1),
            "peak": PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(dom["frac"], 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "avg_us": round(dom["avg_us"], 3),
        },
        "cpu_baseline": cpu,
        "prefill": None if prefill is None else _rounded(prefill),
        "paged": None if paged is None else _rounded(paged),
        "shared": None if shared is None else _rounded(shared),
        "mla": None if mla is None else _rounded(mla),
        "decode_step": None if dstep is None else _rounded(dstep),
        "batches": {str(b): {k: (round(v, 4) if isinstance(v, float) else v)
                             for k, v in r.items() if k not in ("dominant", "kernels_avg_us")}
                    | {"gateup_gbps": round(r["dominant"]["gbps"], 1),
                       "gateup_avg_us": round(r["dominant"]["avg_us"], 3),
                       "kernels_avg_us": {k: round(v, 3) for k, v in r["kernels_avg_us"].items()}}
                    for b, r in results.items()},
    }
    print(json.dumps(line), flush=True)
    cuda.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
