"""ctypes wrapper around oracle/liblp_oracle.so, the CPU restatement of the
reference path.  Test infrastructure: used only as the checker."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PATH = os.path.join(ROOT, "oracle", "liblp_oracle.so")

_lib = None

GATING_SOFTMAX = 0
GATING_SIGMOID = 1


class Layer(C.Structure):
    _fields_ = [
        ("hidden", C.c_int), ("inter", C.c_int), ("experts", C.c_int), ("top_k", C.c_int),
        ("group", C.c_int), ("gating", C.c_int), ("renorm", C.c_int),
        ("routed_scaling", C.c_float), ("min_weight", C.c_float),
        ("router_w", C.c_void_p), ("router_bias", C.c_void_p), ("blobs", C.c_void_p),
        ("gate_off", C.c_uint64), ("up_off", C.c_uint64), ("down_off", C.c_uint64),
        ("shared_blob", C.c_void_p), ("shared_inter", C.c_int), ("shared_group", C.c_int),
        ("sh_gate_off", C.c_uint64), ("sh_up_off", C.c_uint64), ("sh_down_off", C.c_uint64),
    ]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(PATH):
            import subprocess
            subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
        L = C.CDLL(PATH)
        vp, i32, f32, u64, sz = C.c_void_p, C.c_int, C.c_float, C.c_uint64, C.c_size_t
        sigs = {
            "lpo_f32_to_f16_ref": (C.c_uint16, [f32]),
            "lpo_f16_to_f32": (f32, [C.c_uint16]),
            "lpo_bf16_to_f32": (f32, [C.c_uint16]),
            "lpo_expf": (f32, [f32]),
            "lpo_expf_sweep": (None, [C.c_uint32, C.c_uint32, sz, vp]),
            "lpo_q4_bytes": (sz, [sz, sz, sz]),
            "lpo_q4_quantize": (i32, [vp, sz, sz, sz, vp, sz, C.POINTER(f32)]),
            "lpo_q4_store_group": (None, [vp, sz, sz, sz, sz, sz, f32, vp]),
            "lpo_q4_dequantize": (i32, [vp, sz, sz, sz, sz, vp]),
            "lpo_q4_gemv": (None, [vp, vp, vp, i32, i32, i32]),
            "lpo_q4_gemv_batch": (None, [vp, u64, vp, i32, vp, i32, i32, i32, i32]),
            "lpo_bf16_gemv": (None, [vp, vp, vp, i32, i32]),
            "lpo_silu_mul": (None, [vp, vp, vp, i32]),
            "lpo_moe_reduce": (None, [vp, vp, vp, i32, i32]),
            "lpo_add": (None, [vp, vp, i32]),
            "lpo_top_k_softmax": (i32, [vp, i32, i32, i32, vp, vp]),
            "lpo_sigmoid_topk": (i32, [vp, vp, i32, i32, i32, f32, f32, vp, vp]),
            "lpo_router_logits": (None, [vp, vp, vp, i32, i32]),
            "lpo_moe_dispatch": (i32, [vp, vp, i32, i32, i32, vp, vp, vp, vp]),
            "lpo_moe_layer": (i32, [C.POINTER(Layer), vp, vp, i32, vp, vp, vp, vp, vp, i32, i32]),
            "lpo_f32_to_f16_rne": (C.c_uint16, [f32]),
            "lpo_rmsnorm": (None, [vp, vp, vp, i32, i32, f32]),
            "lpo_scale_add": (None, [vp, vp, f32, i32]),
            "lpo_kv_append": (None, [vp, vp, vp, vp, i32, i32, i32, i32, i32]),
            "lpo_rope": (None, [vp, i32, i32, i32, f32]),
            "lpo_attn_decode": (None, [vp, vp, vp, vp, i32, i32, i32, i32, i32, f32, i32]),
            "lpo_bf16_row": (None, [vp, i32, i32, vp]),
            "lpo_mla_rope": (None, [vp, i32, i32, i32, i32, i32, vp, f32]),
            "lpo_mla_attn_decode": (None, [vp, vp, i32, vp, i32, i32, i32, i32, f32, i32]),
            "lpo_bf16_gemv_batch": (None, [vp, u64, vp, i32, vp, i32, i32, i32, i32]),
            "lpo_strided_copy": (None, [vp, i32, i32, vp, i32, i32, i32, i32]),
        }
        for n, (r, a) in sigs.items():
            fn = getattr(L, n)
            fn.restype = r
            fn.argtypes = a
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def f32_to_f16_ref(x: float) -> int:
    return lib().lpo_f32_to_f16_ref(x)


def f16_to_f32(h: int) -> float:
    return lib().lpo_f16_to_f32(h)


def expf(x: float) -> float:
    return lib().lpo_expf(x)


def expf_sweep(first: int, stride: int, n: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    lib().lpo_expf_sweep(first, stride, n, out.ctypes.data)
    return out


def q4_bytes(rows, cols, group):
    return lib().lpo_q4_bytes(rows, cols, group)


def q4_quantize(src: np.ndarray, rows, cols, group):
    src = np.ascontiguousarray(src, np.float32)
    dst = np.zeros(q4_bytes(rows, cols, group), np.uint8)
    err = C.c_float()
    rc = lib().lpo_q4_quantize(_p(src), rows, cols, group, _p(dst), dst.size, C.byref(err))
    if rc != 0:
        raise ValueError("bad dimensions")
    return dst, err.value


def q4_dequantize(buf: np.ndarray, rows, cols, group):
    out = np.zeros(rows * cols, np.float32)
    rc = lib().lpo_q4_dequantize(_p(buf), buf.size, rows, cols, group, _p(out))
    if rc != 0:
        raise ValueError("bad dimensions")
    return out.reshape(rows, cols)


def q4_store_group(dst, rows, cols, group, row, g, scale, qs):
    qs = np.ascontiguousarray(qs, np.uint8)
    lib().lpo_q4_store_group(_p(dst), rows, cols, group, row, g, scale, _p(qs))


def q4_gemv(region: np.ndarray, x: np.ndarray, rows, cols, group):
    y = np.zeros(rows, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    lib().lpo_q4_gemv(_p(region), _p(x), _p(y), rows, cols, group)
    return y


def bf16_gemv(w: np.ndarray, x: np.ndarray, rows, cols):
    y = np.zeros(rows, np.float32)
    lib().lpo_bf16_gemv(_p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(x, np.float32)),
                        _p(y), rows, cols)
    return y


def silu_mul(g, u):
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.zeros_like(g)
    lib().lpo_silu_mul(_p(g), _p(u), _p(out), g.size)
    return out


def moe_reduce(eouts, wts, out):
    out = np.array(out, np.float32, copy=True)
    eo = np.ascontiguousarray(eouts, np.float32)
    w = np.ascontiguousarray(wts, np.float32)
    lib().lpo_moe_reduce(_p(eo), _p(w), _p(out), w.size, out.size)
    return out


def add(a, b):
    a = np.array(a, np.float32, copy=True)
    lib().lpo_add(_p(a), _p(np.ascontiguousarray(b, np.float32)), a.size)
    return a


def top_k_softmax(logits, k, renorm):
    lg = np.ascontiguousarray(logits, np.float32)
    ids = np.zeros(k, np.int32)
    w = np.zeros(k, np.float32)
    n = lib().lpo_top_k_softmax(_p(lg), lg.size, k, int(renorm), _p(ids), _p(w))
    return ids[:n], w[:n]


def sigmoid_topk(logits, bias, k, renorm, scaling, min_weight):
    lg = np.ascontiguousarray(logits, np.float32)
    b = np.ascontiguousarray(bias, np.float32)
    ids = np.zeros(k, np.int32)
    w = np.zeros(k, np.float32)
    n = lib().lpo_sigmoid_topk(_p(lg), _p(b), lg.size, k, int(renorm), scaling, min_weight,
                               _p(ids), _p(w))
    return ids[:n], w[:n]


def router_logits(w_bf16: np.ndarray, x: np.ndarray, E, H):
    out = np.zeros(E, np.float32)
    lib().lpo_router_logits(_p(np.ascontiguousarray(w_bf16, np.uint16)),
                            _p(np.ascontiguousarray(x, np.float32)), _p(out), E, H)
    return out


def moe_dispatch(ids: np.ndarray, cnt: np.ndarray, T, k, E):
    ids = np.ascontiguousarray(ids, np.int32)
    cnt = np.ascontiguousarray(cnt, np.int32)
    perm = np.full(T * k, -1, np.int32)
    gs = np.zeros(E + 1, np.int32)
    inv = np.full(T * k, -1, np.int32)
    uniq = np.zeros(E, np.int32)
    nu = lib().lpo_moe_dispatch(_p(ids), _p(cnt), T, k, E, _p(perm), _p(gs), _p(inv), _p(uniq))
    P = int(gs[E])
    return perm[:P], gs, inv, uniq[:nu]


def moe_layer(desc: dict, blobs: list, x: np.ndarray, h: np.ndarray, logits_in=None, wave=0,
              threads=1, shared_blob=None):
    """One layer.  desc has hidden/inter/experts/top_k/group/gating/renorm/
    routed_scaling/min_weight/router_w (uint16)/router_bias; blobs is a list of
    E uint8 arrays or None.  Returns (h_out, logits, ids, w, cnt)."""
    H, I, E, k = desc["hidden"], desc["inter"], desc["experts"], desc["top_k"]
    T = x.shape[0]
    ptrs = (C.c_void_p * E)(*[(b.ctypes.data if b is not None else None) for b in blobs])
    go, uo, do = desc["offsets"]
    L = Layer(hidden=H, inter=I, experts=E, top_k=k, group=desc["group"],
              gating=desc.get("gating", 0), renorm=int(desc.get("renorm", 1)),
              routed_scaling=desc.get("routed_scaling", 1.0), min_weight=desc.get("min_weight", 0.0),
              router_w=_p(desc["router_w"]), router_bias=_p(desc.get("router_bias")),
              blobs=C.cast(ptrs, C.c_void_p), gate_off=go, up_off=uo, down_off=do)
    if shared_blob is not None:
        L.shared_blob = shared_blob["blob"].ctypes.data
        L.shared_inter = shared_blob["inter"]
        L.shared_group = shared_blob["group"]
        L.sh_gate_off, L.sh_up_off, L.sh_down_off = shared_blob["offsets"]
    hout = np.array(h, np.float32, copy=True)
    x = np.ascontiguousarray(x, np.float32)
    logits = np.zeros((T, E), np.float32)
    ids = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    cnt = np.zeros(T, np.int32)
    li = None if logits_in is None else np.ascontiguousarray(logits_in, np.float32)
    rc = lib().lpo_moe_layer(C.byref(L), _p(x), _p(hout), T, _p(li), _p(logits), _p(ids), _p(w),
                             _p(cnt), wave, threads)
    if rc != 0:
        raise RuntimeError("oracle: routed expert without a blob")
    return hout, logits, ids, w, cnt


# ---- the rest of the decode step and MLA (kernels_bench.rs CPU forms) --------

def f32_to_f16_rne(x: float) -> int:
    return lib().lpo_f32_to_f16_rne(x)


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def rmsnorm(x, w, rows, n, eps):
    x, w = _f32(x), _f32(w)
    y = np.zeros(rows * n, np.float32)
    lib().lpo_rmsnorm(_p(x), _p(w), _p(y), rows, n, eps)
    return y


def scale_add(a, b, s):
    a = np.array(a, np.float32, copy=True)
    lib().lpo_scale_add(_p(a), _p(_f32(b)), s, a.size)
    return a


def kv_append(k, v, kcache, vcache, kv_heads, head_dim, pos, max_seq, f16):
    kc, vc = np.array(kcache, copy=True), np.array(vcache, copy=True)
    lib().lpo_kv_append(_p(_f32(k)), _p(_f32(v)), _p(kc), _p(vc), kv_heads, head_dim, pos, max_seq, int(f16))
    return kc, vc


def rope(x, heads, head_dim, pos, base):
    x = np.array(x, np.float32, copy=True)
    lib().lpo_rope(_p(x), heads, head_dim, pos, base)
    return x


def attn_decode(q, kcache, vcache, heads, kv_heads, head_dim, seq_len, max_seq, scale, f16):
    out = np.zeros(heads * head_dim, np.float32)
    lib().lpo_attn_decode(_p(_f32(q)), _p(np.ascontiguousarray(kcache)), _p(np.ascontiguousarray(vcache)), _p(out),
                          heads, kv_heads, head_dim, seq_len, max_seq, scale, int(f16))
    return out


def bf16_row(table, row, n):
    out = np.zeros(n, np.float32)
    lib().lpo_bf16_row(_p(np.ascontiguousarray(table, np.uint16)), row, n, _p(out))
    return out


def mla_rope(x, n_vecs, stride, offset, half, pos, inv_freq, mscale):
    x = np.array(x, np.float32, copy=True)
    lib().lpo_mla_rope(_p(x), n_vecs, stride, offset, half, pos, _p(_f32(inv_freq)), mscale)
    return x


def mla_attn_decode(q, cache, heads, qk_dim, c_dim, seq_len, scale, bf16=False, threads=8):
    ctx = np.zeros(heads * c_dim, np.float32)
    c = np.ascontiguousarray(cache, np.uint16 if bf16 else np.float32)
    lib().lpo_mla_attn_decode(_p(_f32(q)), _p(c), int(bf16), _p(ctx), heads, qk_dim, c_dim, seq_len, scale,
                              threads)
    return ctx


def bf16_gemv_batch(w, w_stride, x, x_stride, y_stride, rows, cols, batch):
    y = np.zeros(max(1, (batch - 1) * y_stride + rows), np.float32)
    lib().lpo_bf16_gemv_batch(_p(np.ascontiguousarray(w, np.uint16)), w_stride, _p(_f32(x)), x_stride, _p(y),
                              y_stride, rows, cols, batch)
    return y


def strided_copy(src, src_stride, src_off, dst, dst_stride, dst_off, n_vecs, n):
    dst = np.array(dst, np.float32, copy=True)
    lib().lpo_strided_copy(_p(_f32(src)), src_stride, src_off, _p(dst), dst_stride, dst_off, n_vecs, n)
    return dst
