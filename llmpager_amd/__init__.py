"""llmpager_amd -- MI355X (gfx950) MoE-layer hot path of glennswest/llmpager.

The product is the C-ABI library ``lib/libllmpager_hip.so`` (include/llmpager_hip.h)
and the gfx950 code objects it loads.  This module is a thin ctypes binding
whose classes mirror the reference crate's surfaces:

  Cuda     driver::Cuda        (crates/llmpager-cuda/src/driver.rs)
  Kernels  kernels::Kernels    (crates/llmpager-cuda/src/kernels.rs), hot-path methods
  MoeLayer the fused layer: router, top-k, dispatch, grouped experts, combine

There is no CPU fallback: if the library or a code object is missing, loading
raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBDIR = os.path.join(HERE, "lib")
LIBPATH = os.path.join(LIBDIR, "libllmpager_hip.so")

GATING_SOFTMAX = 0
GATING_SIGMOID = 1

_lib = None


class DevPtr(int):
    """A device address (an int, as the C ABI takes it) that remembers the
    size of its allocation, so entry points that need a buffer's size (the
    workspace) can pass it on."""

    def __new__(cls, addr: int, nbytes: int):
        o = super().__new__(cls, addr)
        o.nbytes = int(nbytes)
        return o


class LpError(RuntimeError):
    """A non-zero return from the C ABI, with lp_last_error()'s text."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"llmpager_hip error {code}: {msg}")
        self.code = code


class LayerDesc(C.Structure):
    """lp_moe_layer_desc (include/llmpager_hip.h)."""

    _fields_ = [
        ("hidden", C.c_int32), ("inter", C.c_int32), ("experts", C.c_int32),
        ("top_k", C.c_int32), ("group", C.c_int32), ("gating", C.c_int32),
        ("renorm", C.c_int32), ("routed_scaling", C.c_float), ("min_weight", C.c_float),
        ("reserved0", C.c_int32),
        ("router_w", C.c_uint64), ("router_bias", C.c_uint64), ("slot_table", C.c_uint64),
        ("arena_base", C.c_uint64), ("slot_span", C.c_uint64),
        ("gate_off", C.c_uint64), ("up_off", C.c_uint64), ("down_off", C.c_uint64),
        ("shared_blob", C.c_uint64), ("shared_inter", C.c_int32), ("shared_group", C.c_int32),
        ("sh_gate_off", C.c_uint64), ("sh_up_off", C.c_uint64), ("sh_down_off", C.c_uint64),
    ]


class WsLayout(C.Structure):
    """lp_moe_ws_layout: byte offsets of the workspace parts."""

    _fields_ = [(n, C.c_uint64) for n in (
        "logits", "ids", "wts", "cnt", "gs", "perm", "inv", "uniq", "meta", "et", "act", "y", "xf", "xd",
        "sh_et", "sh_perm", "sh_act", "sh_y", "tiles", "actimg", "xexp", "disp", "total")]


def _sig(lib):
    u64, i32, f32, vp = C.c_uint64, C.c_int, C.c_float, C.c_void_p
    P = C.POINTER
    sigs = {
        "lp_last_error": (C.c_char_p, []),
        "lp_version": (C.c_char_p, []),
        "lp_init": (i32, [i32, C.c_char_p, P(vp)]),
        "lp_destroy": (None, [vp]),
        "lp_bind_thread": (i32, [vp]),
        "lp_mem_info": (i32, [vp, P(u64), P(u64)]),
        "lp_alloc_device": (i32, [vp, C.c_size_t, P(u64)]),
        "lp_free_device": (i32, [vp, u64]),
        "lp_alloc_pinned": (i32, [vp, C.c_size_t, P(vp)]),
        "lp_free_pinned": (i32, [vp, vp]),
        "lp_stream_create": (i32, [vp, P(vp)]),
        "lp_stream_destroy": (i32, [vp, vp]),
        "lp_event_create": (i32, [vp, P(vp)]),
        "lp_event_destroy": (i32, [vp, vp]),
        "lp_htod_async": (i32, [vp, u64, vp, C.c_size_t, vp]),
        "lp_dtoh_async": (i32, [vp, vp, u64, C.c_size_t, vp]),
        "lp_dtod_async": (i32, [vp, u64, u64, C.c_size_t, vp]),
        "lp_memset_async": (i32, [vp, u64, i32, C.c_size_t, vp]),
        "lp_record_event": (i32, [vp, vp, vp]),
        "lp_sync_event": (i32, [vp, vp]),
        "lp_event_done": (i32, [vp, vp]),
        "lp_event_elapsed_ms": (i32, [vp, vp, vp, P(f32)]),
        "lp_stream_wait_event": (i32, [vp, vp, vp]),
        "lp_sync_stream": (i32, [vp, vp]),
        "lp_sync": (i32, [vp]),
        "lp_q4_gemv_batch": (i32, [vp, u64, u64, u64, i32, u64, i32, i32, i32, i32, vp]),
        "lp_q4_gemv": (i32, [vp, u64, u64, u64, i32, i32, i32, vp]),
        "lp_moe_reduce": (i32, [vp, u64, u64, u64, i32, i32, vp]),
        "lp_silu_mul": (i32, [vp, u64, u64, u64, i32, vp]),
        "lp_bf16_gemv": (i32, [vp, u64, u64, u64, i32, i32, vp]),
        "lp_add": (i32, [vp, u64, u64, i32, vp]),
        "lp_rmsnorm": (i32, [vp, u64, u64, u64, i32, i32, f32, vp]),
        "lp_scale_add": (i32, [vp, u64, u64, f32, i32, vp]),
        "lp_kv_append": (i32, [vp, u64, u64, u64, u64, i32, i32, i32, i32, i32, vp]),
        "lp_rope": (i32, [vp, u64, i32, i32, i32, f32, vp]),
        "lp_attn_decode": (i32, [vp, u64, u64, u64, u64, u64, i32, i32, i32, i32, i32, f32, i32, vp]),
        "lp_bf16_row": (i32, [vp, u64, i32, i32, u64, vp]),
        "lp_rmsnorm_gemv": (i32, [vp, u64, u64, f32, i32, u64, i32, u64, u64, i32, u64, u64, i32, u64, vp]),
        "lp_gemv_add_rmsnorm": (i32, [vp, u64, u64, i32, i32, u64, u64, f32, u64, vp]),
        "lp_attn_fused": (i32, [vp, u64, u64, u64, u64, u64, f32, f32, u64, u64, u64, u64, i32, i32, i32, i32, i32,
                                f32, vp]),
        "lp_attn_block": (i32, [vp, u64, u64, u64, u64, u64, f32, f32, u64, u64, u64, u64, i32, i32, i32, i32, i32,
                                f32, u64, u64, u64, u64, i32, vp]),
        "lp_step_errors_sync": (i32, [vp, P(i32)]),
        "lp_mla_rope": (i32, [vp, u64, i32, i32, i32, i32, i32, u64, f32, vp]),
        "lp_mla_attn_decode": (i32, [vp, u64, u64, u64, u64, i32, i32, i32, i32, i32, f32, vp]),
        "lp_bf16_gemv_batch": (i32, [vp, u64, u64, u64, i32, u64, i32, i32, i32, i32, vp]),
        "lp_strided_copy": (i32, [vp, u64, i32, i32, u64, i32, i32, i32, i32, vp]),
        "lp_mla_batch_ws_bytes": (u64, [vp, i32, i32, i32]),
        "lp_mla_attn_decode_batch": (i32, [vp, u64, u64, u64, u64, u64, u64, i32, i32, i32, i32, i32, f32, vp]),
        "lp_moe_ws_layout_get": (i32, [P(LayerDesc), i32, P(WsLayout)]),
        "lp_moe_workspace_check": (i32, [P(LayerDesc), i32, i32, u64, u64]),
        "lp_moe_route": (i32, [vp, P(LayerDesc), u64, i32, u64, u64, vp]),
        "lp_moe_route_logits": (i32, [vp, P(LayerDesc), u64, i32, u64, u64, vp]),
        "lp_moe_experts": (i32, [vp, P(LayerDesc), u64, u64, i32, u64, u64, vp]),
        "lp_moe_experts_wave": (i32, [vp, P(LayerDesc), u64, u64, i32, u64, u64, i32, i32, i32, vp]),
        "lp_moe_resolve": (i32, [vp, P(LayerDesc), i32, u64, u64, vp]),
        "lp_moe_forward": (i32, [vp, P(LayerDesc), u64, u64, i32, u64, u64, vp]),
        "lp_moe_forward_noalloc": (i32, [vp, P(LayerDesc), u64, u64, i32, vp]),
        "lp_moe_stack_forward": (i32, [vp, P(LayerDesc), i32, u64, i32, u64, u64, vp]),
        "lp_moe_stack_capture": (i32, [vp, P(LayerDesc), i32, u64, i32, u64, u64, vp, P(vp)]),
        "lp_graph_capture_begin": (i32, [vp, vp]),
        "lp_graph_capture_end": (i32, [vp, vp, P(vp)]),
        "lp_graph_launch": (i32, [vp, vp, vp]),
        "lp_graph_destroy": (None, [vp]),
        "lp_noalloc_scratch_bytes": (u64, []),
        "lp_moe_status_sync": (i32, [vp, u64, u64, P(LayerDesc), i32, vp, P(C.c_int32), P(C.c_int32)]),
        "lp_q4_bytes": (u64, [i32, i32, i32]),
        "lp_blob_bytes": (u64, [i32, i32, i32]),
        "lp_blob_offsets": (None, [i32, i32, i32, P(u64), P(u64), P(u64)]),
        "lp_synth_blob": (i32, [vp, i32, i32, i32, u64, i32, i32]),
        "lp_synth_blobs": (i32, [vp, u64, i32, i32, i32, i32, u64, i32, i32, i32]),
        "lp_synth_bf16": (i32, [vp, u64, f32, u64, u64]),
        "lp_synth_f32_bf16": (i32, [vp, u64, f32, u64, u64]),
        "lp_profile_enable": (i32, [vp, i32]),
        "lp_profile_reset": (i32, [vp]),
        "lp_profile_read_sync": (i32, [vp, C.c_char_p, P(C.c_double), P(C.c_int64)]),
        "lp_route_expf": (f32, [f32]),
        "lp_route_expf_sweep": (None, [C.c_uint32, C.c_uint32, u64, vp]),
        "lp_route_expf_device": (i32, [vp, C.c_uint32, C.c_uint32, u64, u64, vp]),
        "lp_pager_new": (i32, [vp, vp, P(vp)]),
        "lp_pager_open": (i32, [vp, C.c_char_p, vp, P(vp)]),
        "lp_pager_request_handles": (i32, [vp, C.c_uint16, vp, i32, vp]),
        "lp_pager_wait_stream": (i32, [vp, vp, vp]),
        "lp_pager_refresh_table": (i32, [vp, C.c_uint16, vp]),
        "lp_pager_expert_stats": (i32, [vp, vp, u64]),
        "lp_pager_prewarm": (i32, [vp, vp, u64]),
        "lp_pack_create": (i32, [C.c_char_p, C.c_char_p, C.c_char_p, C.c_uint32, C.c_uint32, P(vp)]),
        "lp_pack_add_blob": (i32, [vp, vp, u64]),
        "lp_pack_finish": (i32, [vp]),
        "lp_pack_open": (i32, [C.c_char_p, i32, P(vp)]),
        "lp_pack_close": (None, [vp]),
        "lp_pack_info": (i32, [vp, P(C.c_uint32), P(C.c_uint32), P(u64)]),
        "lp_pack_entry": (i32, [vp, C.c_uint32, C.c_uint32, P(u64), P(u64)]),
        "lp_pack_read_blob": (C.c_int64, [vp, C.c_uint32, C.c_uint32, vp, u64]),
        "lp_pager_free": (None, [vp]),
        "lp_pager_arena": (u64, [vp]),
        "lp_pager_span": (u64, [vp]),
        "lp_pager_slot_table": (u64, [vp, C.c_uint32]),
        "lp_pager_slots_per_layer": (C.c_uint32, [vp]),
        "lp_pager_request": (i32, [vp, C.c_uint16, vp, i32, vp, vp]),
        "lp_pager_release": (i32, [vp, vp, i32]),
        "lp_pager_release_after": (i32, [vp, vp, i32, vp]),
        "lp_pager_prefetch": (i32, [vp, C.c_uint16, vp, i32]),
        "lp_pager_wait": (i32, [vp, C.c_uint32]),
        "lp_pager_tick": (i32, [vp]),
        "lp_pager_sync": (i32, [vp]),
        "lp_pager_get_metrics": (i32, [vp, vp]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def lib() -> C.CDLL:
    """The loaded C-ABI library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBPATH):
            raise RuntimeError(
                f"{LIBPATH} is missing: build it with `python -m llmpager_amd.build` "
                "(there is no CPU fallback)")
        _lib = _sig(C.CDLL(LIBPATH))
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        raise LpError(rc, lib().lp_last_error().decode())


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# ---- host-only helpers (no device needed) ----------------------------------

def q4_bytes(rows: int, cols: int, group: int) -> int:
    return int(lib().lp_q4_bytes(rows, cols, group))


def blob_bytes(hidden: int, inter: int, group: int) -> int:
    return int(lib().lp_blob_bytes(hidden, inter, group))


def blob_offsets(hidden: int, inter: int, group: int) -> tuple[int, int, int]:
    g, u, d = C.c_uint64(), C.c_uint64(), C.c_uint64()
    lib().lp_blob_offsets(hidden, inter, group, C.byref(g), C.byref(u), C.byref(d))
    return g.value, u.value, d.value


def synth_blob(hidden: int, inter: int, group: int, seed: int, layer: int, expert: int) -> np.ndarray:
    out = np.zeros(blob_bytes(hidden, inter, group), np.uint8)
    _check(lib().lp_synth_blob(_ptr(out), hidden, inter, group, seed, layer, expert))
    return out


def synth_blobs(n: int, stride: int, hidden: int, inter: int, group: int, seed: int, layer: int,
                e0: int = 0, threads: int = 0, out: np.ndarray | None = None) -> np.ndarray:
    if out is None:
        out = np.zeros(n * stride, np.uint8)
    threads = threads or min(16, os.cpu_count() or 1)
    _check(lib().lp_synth_blobs(_ptr(out), stride, n, hidden, inter, group, seed, layer, e0, threads))
    return out


def synth_bf16(n: int, std: float, seed: int, stream: int) -> np.ndarray:
    out = np.zeros(n, np.uint16)
    _check(lib().lp_synth_bf16(_ptr(out), n, std, seed, stream))
    return out


def synth_f32_bf16(n: int, std: float, seed: int, stream: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    _check(lib().lp_synth_f32_bf16(_ptr(out), n, std, seed, stream))
    return out


def route_expf(x: float) -> float:
    return float(lib().lp_route_expf(x))


def route_expf_sweep(first: int, stride: int, n: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    lib().lp_route_expf_sweep(first, stride, n, _ptr(out))
    return out


def dimage_bytes(cols: int) -> int:
    """Bytes of one row's digit image in the workspace's xd part: per padded
    32-column sub-group 32 B of hi digits, 32 B of lo digits, an 8-byte seed
    pair and a 4-byte scale."""
    return 76 * 4 * (((cols >> 5) + 3) >> 2)


def ws_layout(desc: LayerDesc, T: int) -> WsLayout:
    lay = WsLayout()
    _check(lib().lp_moe_ws_layout_get(C.byref(desc), T, C.byref(lay)))
    return lay


# ---- device runtime: driver::Cuda -------------------------------------------

class Cuda:
    """driver::Cuda (driver.rs:29-304) over the C ABI."""

    def __init__(self, device: int = 0, hsaco_dir: str | None = None):
        self.ctx = C.c_void_p()
        d = hsaco_dir.encode() if hsaco_dir else None
        _check(lib().lp_init(device, d, C.byref(self.ctx)))

    def close(self) -> None:
        if self.ctx:
            lib().lp_destroy(self.ctx)
            self.ctx = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def bind_thread(self) -> None:
        _check(lib().lp_bind_thread(self.ctx))

    def mem_info(self) -> tuple[int, int]:
        f, t = C.c_uint64(), C.c_uint64()
        _check(lib().lp_mem_info(self.ctx, C.byref(f), C.byref(t)))
        return f.value, t.value

    def alloc_device(self, nbytes: int) -> "DevPtr":
        p = C.c_uint64()
        _check(lib().lp_alloc_device(self.ctx, nbytes, C.byref(p)))
        return DevPtr(p.value, nbytes)

    def free_device(self, p: int) -> None:
        _check(lib().lp_free_device(self.ctx, p))

    def alloc_pinned(self, nbytes: int) -> int:
        p = C.c_void_p()
        _check(lib().lp_alloc_pinned(self.ctx, nbytes, C.byref(p)))
        return p.value

    def free_pinned(self, p: int) -> None:
        _check(lib().lp_free_pinned(self.ctx, p))

    def stream(self) -> int:
        s = C.c_void_p()
        _check(lib().lp_stream_create(self.ctx, C.byref(s)))
        return s.value

    def destroy_stream(self, s: int) -> None:
        _check(lib().lp_stream_destroy(self.ctx, s))

    def capture_begin(self, s: int) -> None:
        """Record every launch this library makes on stream s (lp_graph_capture_begin)."""
        _check(lib().lp_graph_capture_begin(self.ctx, s))

    def capture_end(self, s: int) -> "Graph":
        """The launches recorded since capture_begin, as one graph (lp_graph_capture_end)."""
        g = C.c_void_p()
        _check(lib().lp_graph_capture_end(self.ctx, s, C.byref(g)))
        return Graph(self, g.value)

    def event(self) -> int:
        e = C.c_void_p()
        _check(lib().lp_event_create(self.ctx, C.byref(e)))
        return e.value

    def destroy_event(self, e: int) -> None:
        _check(lib().lp_event_destroy(self.ctx, e))

    def htod_async(self, dst: int, src: np.ndarray, stream: int | None = None) -> None:
        src = np.ascontiguousarray(src)
        _check(lib().lp_htod_async(self.ctx, dst, _ptr(src), src.nbytes, stream))

    def htod_ptr_async(self, dst: int, src_ptr: int, nbytes: int, stream: int | None = None) -> None:
        _check(lib().lp_htod_async(self.ctx, dst, src_ptr, nbytes, stream))

    def dtoh_async(self, dst: np.ndarray, src: int, stream: int | None = None) -> None:
        assert dst.flags["C_CONTIGUOUS"]
        _check(lib().lp_dtoh_async(self.ctx, _ptr(dst), src, dst.nbytes, stream))

    def dtoh_ptr_async(self, dst_ptr: int, src: int, nbytes: int, stream: int | None = None) -> None:
        _check(lib().lp_dtoh_async(self.ctx, dst_ptr, src, nbytes, stream))

    def dtod_async(self, dst: int, src: int, nbytes: int, stream: int | None = None) -> None:
        _check(lib().lp_dtod_async(self.ctx, dst, src, nbytes, stream))

    def memset_async(self, dst: int, value: int, nbytes: int, stream: int | None = None) -> None:
        _check(lib().lp_memset_async(self.ctx, dst, value, nbytes, stream))

    def record_event(self, e: int, s: int | None = None) -> None:
        _check(lib().lp_record_event(self.ctx, e, s))

    def sync_event(self, e: int) -> None:
        _check(lib().lp_sync_event(self.ctx, e))

    def event_done(self, e: int) -> bool:
        r = lib().lp_event_done(self.ctx, e)
        if r < 0:
            _check(r)
        return r == 1

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = C.c_float()
        _check(lib().lp_event_elapsed_ms(self.ctx, a, b, C.byref(ms)))
        return ms.value

    def stream_wait_event(self, s: int, e: int) -> None:
        _check(lib().lp_stream_wait_event(self.ctx, s, e))

    def sync_stream(self, s: int | None = None) -> None:
        _check(lib().lp_sync_stream(self.ctx, s))

    def sync(self) -> None:
        _check(lib().lp_sync(self.ctx))

    def step_errors(self) -> int:
        """Waits of the fused decode step that gave up since the last call
        (lp_step_errors_sync; 0 normally)."""
        n = C.c_int32()
        _check(lib().lp_step_errors_sync(self.ctx, C.byref(n)))
        return n.value

    # measurement (lp_profile_*)
    def profile(self, enable: bool) -> None:
        _check(lib().lp_profile_enable(self.ctx, int(enable)))

    def profile_reset(self) -> None:
        _check(lib().lp_profile_reset(self.ctx))

    def profile_read(self, kernel: str) -> tuple[float, int]:
        ms, n = C.c_double(), C.c_int64()
        _check(lib().lp_profile_read_sync(self.ctx, kernel.encode(), C.byref(ms), C.byref(n)))
        return ms.value, n.value

    # convenience
    def upload(self, a: np.ndarray, stream: int | None = None) -> int:
        a = np.ascontiguousarray(a)
        p = self.alloc_device(max(a.nbytes, 1))
        self.htod_async(p, a, stream)
        return p

    def download(self, p: int, shape, dtype, stream: int | None = None) -> np.ndarray:
        out = np.empty(shape, dtype)
        self.dtoh_async(out, p, stream)
        self.sync_stream(stream)
        return out


# ---- hot-path launchers: kernels::Kernels --------------------------------------

class Kernels:
    """The hot-path methods of kernels::Kernels (kernels.rs), same argument order."""

    def __init__(self, cuda: Cuda):
        self.cuda = cuda

    def q4g64_gemv_batch(self, blobs: int, region_off: int, x: int, x_stride: int, y: int,
                         rows: int, cols: int, group: int, experts: int, stream=None) -> None:
        _check(lib().lp_q4_gemv_batch(self.cuda.ctx, blobs, region_off, x, x_stride, y, rows,
                                      cols, group, experts, stream))

    def q4g64_gemv(self, blob: int, x: int, y: int, rows: int, cols: int, group: int,
                   stream=None) -> None:
        _check(lib().lp_q4_gemv(self.cuda.ctx, blob, x, y, rows, cols, group, stream))

    def moe_reduce(self, eouts: int, wts: int, out: int, experts: int, n: int, stream=None) -> None:
        _check(lib().lp_moe_reduce(self.cuda.ctx, eouts, wts, out, experts, n, stream))

    def silu_mul(self, gate: int, up: int, out: int, n: int, stream=None) -> None:
        _check(lib().lp_silu_mul(self.cuda.ctx, gate, up, out, n, stream))

    def bf16_gemv(self, w: int, x: int, y: int, rows: int, cols: int, stream=None) -> None:
        _check(lib().lp_bf16_gemv(self.cuda.ctx, w, x, y, rows, cols, stream))

    def add(self, a: int, b: int, n: int, stream=None) -> None:
        _check(lib().lp_add(self.cuda.ctx, a, b, n, stream))

    # the rest of the decode step (kernels.rs, decode.cu)
    def rmsnorm(self, x: int, w: int, y: int, rows: int, n: int, eps: float, stream=None) -> None:
        _check(lib().lp_rmsnorm(self.cuda.ctx, x, w, y, rows, n, eps, stream))

    def scale_add(self, a: int, b: int, s: float, n: int, stream=None) -> None:
        _check(lib().lp_scale_add(self.cuda.ctx, a, b, s, n, stream))

    def kv_append(self, k: int, v: int, kcache: int, vcache: int, kv_heads: int, head_dim: int, pos: int,
                  max_seq: int, f16: bool, stream=None) -> None:
        _check(lib().lp_kv_append(self.cuda.ctx, k, v, kcache, vcache, kv_heads, head_dim, pos, max_seq,
                                  int(f16), stream))

    def rope(self, x: int, heads: int, head_dim: int, pos: int, base: float, stream=None) -> None:
        _check(lib().lp_rope(self.cuda.ctx, x, heads, head_dim, pos, base, stream))

    def attn_decode(self, q: int, kcache: int, vcache: int, out: int, scratch: int, heads: int, kv_heads: int,
                    head_dim: int, seq_len: int, max_seq: int, scale: float, f16: bool, stream=None) -> None:
        _check(lib().lp_attn_decode(self.cuda.ctx, q, kcache, vcache, out, scratch, heads, kv_heads, head_dim,
                                    seq_len, max_seq, scale, int(f16), stream))

    def bf16_row(self, table: int, row: int, n: int, out: int, stream=None) -> None:
        _check(lib().lp_bf16_row(self.cuda.ctx, table, row, n, out, stream))

    # the fused decode step (no kernels.rs counterparts: each is several of
    # the launches above in one, lp_step.hip)
    def rmsnorm_gemv(self, x: int, ln: int, eps: float, cols: int, mats, stream=None) -> None:
        """y_i = W_i . rmsnorm(x, ln) for mats = [(w, rows, y), ...] (one to
        three matrices sharing x; ln = 0: no norm)."""
        m = list(mats) + [(0, 0, 0)] * (3 - len(mats))
        if not 1 <= len(mats) <= 3:
            raise ValueError("rmsnorm_gemv takes one to three matrices")
        _check(lib().lp_rmsnorm_gemv(self.cuda.ctx, x, ln, eps, cols, m[0][0], m[0][1], m[0][2], m[1][0], m[1][1],
                                     m[1][2], m[2][0], m[2][1], m[2][2], stream))

    def gemv_add_rmsnorm(self, w: int, x: int, rows: int, cols: int, h: int, ln: int, eps: float, hn: int,
                         stream=None) -> None:
        """h += W . x, then hn = rmsnorm(h, ln)."""
        _check(lib().lp_gemv_add_rmsnorm(self.cuda.ctx, w, x, rows, cols, h, ln, eps, hn, stream))

    def attn_fused(self, q: int, k: int, v: int, q_norm: int, k_norm: int, eps: float, rope_base: float, kcache: int,
                   vcache: int, out: int, scratch: int, heads: int, kv_heads: int, head_dim: int, pos: int,
                   max_seq: int, scale: float, stream=None) -> None:
        """Per-head q / k RMSNorm, RoPE, the fp16 KV append at pos and GQA
        decode attention over positions 0..pos (q, k, v read only)."""
        _check(lib().lp_attn_fused(self.cuda.ctx, q, k, v, q_norm, k_norm, eps, rope_base, kcache, vcache, out,
                                   scratch, heads, kv_heads, head_dim, pos, max_seq, scale, stream))

    def attn_block(self, q: int, k: int, v: int, q_norm: int, k_norm: int, eps: float, rope_base: float, kcache: int,
                   vcache: int, att: int, scratch: int, heads: int, kv_heads: int, head_dim: int, pos: int,
                   max_seq: int, scale: float, wo: int, h: int, post_ln: int, hn: int, hidden: int,
                   stream=None) -> None:
        """attn_fused into att, then h += W_o . att and hn = rmsnorm(h, post_ln), in one launch."""
        _check(lib().lp_attn_block(self.cuda.ctx, q, k, v, q_norm, k_norm, eps, rope_base, kcache, vcache, att,
                                   scratch, heads, kv_heads, head_dim, pos, max_seq, scale, wo, h, post_ln, hn, hidden,
                                   stream))

    # MLA absorbed decode (kernels.rs, mla.cu)
    def mla_rope(self, x: int, n_vecs: int, stride: int, offset: int, half: int, pos: int, inv_freq: int,
                 mscale: float, stream=None) -> None:
        _check(lib().lp_mla_rope(self.cuda.ctx, x, n_vecs, stride, offset, half, pos, inv_freq, mscale, stream))

    def mla_attn_decode(self, q: int, cache: int, ctx: int, scratch: int, heads: int, qk_dim: int, c_dim: int,
                        seq_len: int, max_seq: int, scale: float, stream=None) -> None:
        _check(lib().lp_mla_attn_decode(self.cuda.ctx, q, cache, ctx, scratch, heads, qk_dim, c_dim, seq_len,
                                        max_seq, scale, stream))

    def bf16_gemv_batch(self, w: int, w_stride: int, x: int, x_stride: int, y: int, y_stride: int, rows: int,
                        cols: int, batch: int, stream=None) -> None:
        _check(lib().lp_bf16_gemv_batch(self.cuda.ctx, w, w_stride, x, x_stride, y, y_stride, rows, cols, batch,
                                        stream))

    def strided_copy(self, src: int, src_stride: int, src_off: int, dst: int, dst_stride: int, dst_off: int,
                     n_vecs: int, n: int, stream=None) -> None:
        _check(lib().lp_strided_copy(self.cuda.ctx, src, src_stride, src_off, dst, dst_stride, dst_off, n_vecs, n,
                                     stream))

    def mla_batch_ws_bytes(self, batch: int, c_dim: int, max_seq: int) -> int:
        return int(lib().lp_mla_batch_ws_bytes(self.cuda.ctx, batch, c_dim, max_seq))

    def mla_attn_decode_batch(self, q: int, cache: int, cache_stride: int, seq_lens: int, ctx: int, ws: int,
                              batch: int, heads: int, qk_dim: int, c_dim: int, max_seq: int, scale: float,
                              stream=None) -> None:
        _check(lib().lp_mla_attn_decode_batch(self.cuda.ctx, q, cache, cache_stride, seq_lens, ctx, ws, batch,
                                              heads, qk_dim, c_dim, max_seq, scale, stream))


# ---- fused MoE layer ----------------------------------------------------------------

class PagerConfig(C.Structure):
    """lp_pager_config (include/llmpager_hip.h)."""

    _fields_ = [
        ("layers", C.c_uint32), ("experts_per_layer", C.c_uint32), ("slots_per_layer", C.c_uint32),
        ("decay_interval", C.c_uint32), ("blob_bytes", C.c_uint64), ("span", C.c_uint64),
        ("host_blobs", C.c_void_p), ("host_stride", C.c_uint64), ("copy_streams", C.c_int32),
        ("global_pool", C.c_int32), ("pool_decay_tokens", C.c_uint32), ("source", C.c_int32),
        ("direct", C.c_int32), ("io_threads", C.c_uint32), ("ring_slots", C.c_uint32),
        ("stage_threads", C.c_uint32), ("ram_bytes", C.c_uint64), ("reserve_bytes", C.c_uint64),
    ]


PAGER_SRC_PINNED, PAGER_SRC_HOST, PAGER_SRC_PACK = 0, 1, 2


class PagerMetrics(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("hits", "misses", "bytes_fetched", "fetches", "stalls", "ram_hits")] + [
        ("latency_ms_buckets", C.c_uint64 * 7)]


class ExpertHandle(C.Structure):
    """lp_expert_handle: pager.rs ExpertHandle {layer, expert, slot, dev, len}."""

    _fields_ = [("layer", C.c_uint16), ("expert", C.c_uint16), ("slot", C.c_uint32), ("dev", C.c_uint64),
                ("len", C.c_uint64)]


class PackWriter:
    """PackWriter (pack.rs:67-150) over lp_pack_create / add_blob / finish."""

    def __init__(self, path: str, layers: int, experts: int, model: str = "synthetic", dtype: str = "q4g32-gud"):
        w = C.c_void_p()
        _check(lib().lp_pack_create(path.encode(), model.encode(), dtype.encode(), layers, experts, C.byref(w)))
        self.w = w.value

    def add_blob(self, blob: np.ndarray) -> None:
        b = np.ascontiguousarray(blob, np.uint8)
        _check(lib().lp_pack_add_blob(self.w, _ptr(b), b.size))

    def finish(self) -> None:
        w, self.w = self.w, None
        _check(lib().lp_pack_finish(w))


class Pack:
    """PackReader (pack.rs:152-260) over lp_pack_open / read_blob."""

    def __init__(self, path: str, direct: bool = False):
        p = C.c_void_p()
        _check(lib().lp_pack_open(path.encode(), int(direct), C.byref(p)))
        self.p = p.value
        L, E, m = C.c_uint32(), C.c_uint32(), C.c_uint64()
        _check(lib().lp_pack_info(self.p, C.byref(L), C.byref(E), C.byref(m)))
        self.layers, self.experts, self.max_blob = L.value, E.value, m.value

    def entry(self, layer: int, expert: int) -> tuple[int, int]:
        o, n = C.c_uint64(), C.c_uint64()
        _check(lib().lp_pack_entry(self.p, layer, expert, C.byref(o), C.byref(n)))
        return o.value, n.value

    def read_blob(self, layer: int, expert: int) -> np.ndarray:
        _, n = self.entry(layer, expert)
        span = (n + 4095) // 4096 * 4096
        raw = np.zeros(span + 4096, np.uint8)
        off = (-raw.ctypes.data) % 4096          # a 4096-aligned view, as O_DIRECT needs
        buf = raw[off:off + span]
        got = lib().lp_pack_read_blob(self.p, layer, expert, _ptr(buf), span)
        if got < 0:
            _check(int(got))
        return buf[:got].copy()

    def close(self) -> None:
        if self.p:
            lib().lp_pack_close(self.p)
            self.p = None


class Pager:
    """pager::Pager (pager.rs) over the C ABI: VRAM expert slots, misses filled
    from pinned host blobs on copy streams."""

    def __init__(self, cuda: "Cuda", cfg: PagerConfig, pack_path: str | None = None):
        self.cuda, self.cfg = cuda, cfg
        p = C.c_void_p()
        if pack_path is None:
            _check(lib().lp_pager_new(cuda.ctx, C.byref(cfg), C.byref(p)))
        else:
            _check(lib().lp_pager_open(cuda.ctx, pack_path.encode(), C.byref(cfg), C.byref(p)))
        self.p = p.value

    def request_handles(self, layer: int, experts) -> list:
        """Pager::request: pins and schedules, returns ExpertHandles at once."""
        ex = np.ascontiguousarray(experts, np.uint16)
        out = (ExpertHandle * max(len(ex), 1))()
        _check(lib().lp_pager_request_handles(self.p, layer, _ptr(ex), len(ex), out))
        return [out[i] for i in range(len(ex))]

    def wait_stream(self, h: ExpertHandle, stream=None) -> None:
        _check(lib().lp_pager_wait_stream(self.p, C.byref(h), stream))

    def refresh_table(self, layer: int, stream=None) -> None:
        _check(lib().lp_pager_refresh_table(self.p, layer, stream))

    def expert_stats(self) -> np.ndarray:
        n = lib().lp_pager_expert_stats(self.p, None, 0)
        if n < 0:
            _check(n)
        out = np.zeros(n, np.uint64)
        r = lib().lp_pager_expert_stats(self.p, _ptr(out), n)
        if r < 0:
            _check(r)
        return out

    def prewarm(self, counts) -> int:
        c = np.ascontiguousarray(counts, np.uint64)
        r = lib().lp_pager_prewarm(self.p, _ptr(c), c.size)
        if r < 0:
            _check(r)
        return r

    @property
    def arena(self) -> int:
        return int(lib().lp_pager_arena(self.p))

    @property
    def span(self) -> int:
        return int(lib().lp_pager_span(self.p))

    def slot_table(self, layer: int) -> int:
        return int(lib().lp_pager_slot_table(self.p, layer))

    @property
    def slots_per_layer(self) -> int:
        """Slots per layer in use (after any reserve_bytes clamp)."""
        return int(lib().lp_pager_slots_per_layer(self.p))

    def request(self, layer: int, experts, stream=None) -> np.ndarray:
        ex = np.ascontiguousarray(experts, np.uint16)
        out = np.zeros(len(ex), np.uint32)
        _check(lib().lp_pager_request(self.p, layer, _ptr(ex), len(ex), stream, _ptr(out)))
        return out

    def release(self, slots) -> None:
        sl = np.ascontiguousarray(slots, np.uint32)
        _check(lib().lp_pager_release(self.p, _ptr(sl), len(sl)))

    def release_after(self, slots, stream=None) -> None:
        sl = np.ascontiguousarray(slots, np.uint32)
        _check(lib().lp_pager_release_after(self.p, _ptr(sl), len(sl), stream))

    def prefetch(self, layer: int, experts) -> None:
        ex = np.ascontiguousarray(experts, np.uint16)
        _check(lib().lp_pager_prefetch(self.p, layer, _ptr(ex), len(ex)))

    def wait(self, slot: int) -> None:
        _check(lib().lp_pager_wait(self.p, slot))

    def tick(self) -> None:
        _check(lib().lp_pager_tick(self.p))

    def sync(self) -> None:
        _check(lib().lp_pager_sync(self.p))

    def metrics(self) -> dict:
        m = PagerMetrics()
        _check(lib().lp_pager_get_metrics(self.p, C.byref(m)))
        out = {n: getattr(m, n) for n, _ in PagerMetrics._fields_}
        out["latency_ms_buckets"] = list(m.latency_ms_buckets)
        return out

    def close(self) -> None:
        if self.p:
            lib().lp_pager_free(self.p)
            self.p = None


def _ws_bytes(ws: int, ws_bytes: int | None) -> int:
    """The workspace's size: given, or carried by a DevPtr from alloc_device."""
    if ws_bytes is not None:
        return ws_bytes
    n = getattr(ws, "nbytes", None)
    if n is None:
        raise TypeError("workspace size unknown: pass ws_bytes or a DevPtr from Cuda.alloc_device")
    return n


def workspace_check(descs, T: int, ws: int, ws_bytes: int) -> int:
    """lp_moe_workspace_check (host only): 0, or the code the entry points
    would return for this workspace."""
    arr = (LayerDesc * len(descs))(*descs)
    return lib().lp_moe_workspace_check(arr, len(descs), T, ws, ws_bytes)


class MoeLayer:
    """The fused layer entry points for one layer descriptor.  `ws` is a
    DevPtr from Cuda.alloc_device (its size travels with it) or an address
    with `ws_bytes` given."""

    def __init__(self, cuda: Cuda, desc: LayerDesc):
        self.cuda = cuda
        self.desc = desc

    def route(self, x: int, T: int, ws: int, stream=None, ws_bytes: int | None = None) -> None:
        _check(lib().lp_moe_route(self.cuda.ctx, C.byref(self.desc), x, T, ws, _ws_bytes(ws, ws_bytes), stream))

    def route_logits(self, logits: int, T: int, ws: int, stream=None, ws_bytes: int | None = None) -> None:
        _check(lib().lp_moe_route_logits(self.cuda.ctx, C.byref(self.desc), logits, T, ws,
                                         _ws_bytes(ws, ws_bytes), stream))

    def resolve(self, T: int, ws: int, stream=None, ws_bytes: int | None = None) -> None:
        _check(lib().lp_moe_resolve(self.cuda.ctx, C.byref(self.desc), T, ws, _ws_bytes(ws, ws_bytes), stream))

    def experts(self, x: int, h: int, T: int, ws: int, stream=None, ws_bytes: int | None = None) -> None:
        _check(lib().lp_moe_experts(self.cuda.ctx, C.byref(self.desc), x, h, T, ws, _ws_bytes(ws, ws_bytes),
                                    stream))

    def forward(self, x: int, h: int, T: int, ws: int, stream=None, ws_bytes: int | None = None) -> None:
        _check(lib().lp_moe_forward(self.cuda.ctx, C.byref(self.desc), x, h, T, ws, _ws_bytes(ws, ws_bytes),
                                    stream))

    def experts_wave(self, x: int, h: int, T: int, ws: int, u_first: int, u_count: int, with_shared: bool,
                     stream=None, ws_bytes: int | None = None) -> None:
        """lp_moe_experts_wave: the routed experts uniq[u_first : u_first +
        u_count] of one wave of a paged union (decode.rs:483-531)."""
        _check(lib().lp_moe_experts_wave(self.cuda.ctx, C.byref(self.desc), x, h, T, ws, _ws_bytes(ws, ws_bytes),
                                         u_first, u_count, int(with_shared), stream))

    def forward_noalloc(self, x: int, h: int, T: int, stream=None) -> None:
        """lp_moe_forward_noalloc: the layer with the library's built-in
        per-device scratch as its workspace (no allocation)."""
        _check(lib().lp_moe_forward_noalloc(self.cuda.ctx, C.byref(self.desc), x, h, T, stream))

    def status(self, ws: int, T: int, stream=None, ws_bytes: int | None = None) -> tuple[int, int]:
        u, e = C.c_int32(), C.c_int32()
        _check(lib().lp_moe_status_sync(self.cuda.ctx, ws, _ws_bytes(ws, ws_bytes), C.byref(self.desc), T, stream,
                                        C.byref(u), C.byref(e)))
        return u.value, e.value


class MoeStack:
    """The layer-stack driver (lp_moe_stack_forward): MoE layers in order over
    one residual buffer, the layer input being the residual itself; `capture`
    records the same launches into a replayable HIP graph."""

    def __init__(self, cuda: Cuda, descs):
        self.cuda = cuda
        self.descs = (LayerDesc * len(descs))(*descs)
        self.n = len(descs)

    def ws_bytes(self, T: int) -> int:
        return max(ws_layout(d, T).total for d in self.descs)

    def forward(self, h: int, T: int, ws: int, stream=None, ws_bytes: int | None = None) -> None:
        _check(lib().lp_moe_stack_forward(self.cuda.ctx, self.descs, self.n, h, T, ws, _ws_bytes(ws, ws_bytes),
                                          stream))

    def capture(self, h: int, T: int, ws: int, stream, ws_bytes: int | None = None) -> "Graph":
        g = C.c_void_p()
        _check(lib().lp_moe_stack_capture(self.cuda.ctx, self.descs, self.n, h, T, ws, _ws_bytes(ws, ws_bytes),
                                          stream, C.byref(g)))
        return Graph(self.cuda, g.value)


class Graph:
    """An instantiated HIP graph (lp_graph)."""

    def __init__(self, cuda: Cuda, g: int):
        self.cuda, self.g = cuda, g

    def launch(self, stream) -> None:
        _check(lib().lp_graph_launch(self.cuda.ctx, self.g, stream))

    def close(self) -> None:
        if self.g:
            lib().lp_graph_destroy(self.g)
            self.g = None
