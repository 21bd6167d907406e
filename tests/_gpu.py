"""Helpers for the GPU parity tests: a synthetic MoE layer resident in a slot
arena on the device, plus the matching host copies for the oracle."""
from __future__ import annotations

import numpy as np

import llmpager_amd as lp


def align(v: int, a: int = 4096) -> int:
    return (v + a - 1) // a * a


class DeviceLayer:
    """E synthetic experts of one layer in a device slot arena (slot e =
    expert e, the order a fresh cache hands slots out, cache.rs:142-157)."""

    def __init__(self, cuda: lp.Cuda, H: int, I: int, E: int, k: int, group: int, seed: int = 0,
                 layer: int = 0, gating: int = lp.GATING_SOFTMAX, renorm: bool = True,
                 routed_scaling: float = 1.0, min_weight: float = 0.0, router_std: float = 0.02,
                 bias: np.ndarray | None = None, slots: np.ndarray | None = None,
                 shared: tuple[int, int] | None = None):
        self.cuda = cuda
        self.H, self.I, self.E, self.k, self.group = H, I, E, k, group
        self.blob_bytes = lp.blob_bytes(H, I, group)
        self.span = align(self.blob_bytes)
        self.offsets = lp.blob_offsets(H, I, group)
        self.host = lp.synth_blobs(E, self.span, H, I, group, seed, layer)
        self.arena = cuda.upload(self.host)
        self.router_w = lp.synth_bf16(E * H, router_std, seed, 1000 + layer)
        self.d_router = cuda.upload(self.router_w)
        self.bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self.d_bias = cuda.upload(self.bias) if self.bias is not None else 0
        self.slots = np.arange(E, dtype=np.int32) if slots is None else np.asarray(slots, np.int32)
        self.d_slots = cuda.upload(self.slots)
        self.gating, self.renorm = gating, renorm
        self.routed_scaling, self.min_weight = routed_scaling, min_weight
        go, uo, do = self.offsets
        self.desc = lp.LayerDesc(
            hidden=H, inter=I, experts=E, top_k=k, group=group, gating=gating,
            renorm=int(renorm), routed_scaling=routed_scaling, min_weight=min_weight,
            router_w=self.d_router, router_bias=self.d_bias, slot_table=self.d_slots,
            arena_base=self.arena, slot_span=self.span, gate_off=go, up_off=uo, down_off=do)
        # the always-on shared MLP (kimi.rs:739-744, 779): (inter, group) or None
        self.shared = None
        if shared is not None:
            si, sg = shared
            blob = lp.synth_blob(H, si, sg, seed, layer, 1 << 20)
            self.shared = dict(blob=blob, inter=si, group=sg, offsets=lp.blob_offsets(H, si, sg))
            self.d_shared = cuda.upload(blob)
            self.desc.shared_blob = self.d_shared
            self.desc.shared_inter, self.desc.shared_group = si, sg
            self.desc.sh_gate_off, self.desc.sh_up_off, self.desc.sh_down_off = self.shared["offsets"]
        self.layer = lp.MoeLayer(cuda, self.desc)
        cuda.sync()

    def blob(self, e: int) -> np.ndarray:
        return self.host[e * self.span: e * self.span + self.blob_bytes]

    def oracle_desc(self) -> dict:
        return dict(hidden=self.H, inter=self.I, experts=self.E, top_k=self.k, group=self.group,
                    gating=self.gating, renorm=self.renorm, routed_scaling=self.routed_scaling,
                    min_weight=self.min_weight, router_w=self.router_w, router_bias=self.bias,
                    offsets=self.offsets)

    def oracle_blobs(self) -> list:
        # The oracle sees each expert through the same slot table.
        return [self.blob(int(self.slots[e])) if self.slots[e] >= 0 else None for e in range(self.E)]

    def free(self) -> None:
        for p in (self.arena, self.d_router, self.d_slots):
            self.cuda.free_device(p)
        if self.d_bias:
            self.cuda.free_device(self.d_bias)
        if self.shared is not None:
            self.cuda.free_device(self.d_shared)


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    d = np.linalg.norm(a - b)
    n = np.linalg.norm(b)
    return float(d / n) if n > 0 else float(d)


def worst_rel(got: np.ndarray, want: np.ndarray) -> float:
    """gemv_bench.rs:61-65 / kernels_bench.rs:48-58: max |a-b| / max(|ref|, 1)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want) / np.maximum(np.abs(want), 1.0))) if want.size else 0.0
