"""CPU checks of the C-ABI library: it loads, exports every declared entry
point, and its host-only parts (blob format, synthetic inputs, the routing
expf, descriptor layout, error reporting) behave -- no device calls."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import llmpager_amd as lp
import _oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "llmpager_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lp_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) > 40
    lib = C.CDLL(lp.LIBPATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_code_objects_hold_every_kernel_the_runtime_loads():
    src = open(os.path.join(ROOT, "llmpager_amd", "csrc", "lp_runtime.cpp")).read()
    specs = re.findall(r'\{"(lp_[a-z_]+\.hsaco)", "(lp_[a-z0-9_]+)"\}', src)
    assert len(specs) >= 10
    for module, kernel in specs:
        data = open(os.path.join(lp.LIBDIR, module), "rb").read()
        # an ELF code object, or hipcc's offload bundle wrapping one
        assert data[:4] == b"\x7fELF" or data.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
        assert b"gfx950" in data
        assert kernel.encode() in data, (module, kernel)


def test_version_and_init_error_without_device():
    assert b"gfx950" in lp.lib().lp_version()
    ctx = C.c_void_p()
    rc = lp.lib().lp_init(0, None, C.byref(ctx))
    if rc == 0:  # a device is present: nothing to check here
        lp.lib().lp_destroy(ctx)
        pytest.skip("a GPU is present")
    assert rc != 0 and not ctx
    assert lp.lib().lp_last_error()


def test_blob_format_matches_converter():
    # convert/src/lib.rs:448-471 (H128/I64 at group 64) and decode.rs:161-185
    H, I, g = 128, 64, 64
    assert lp.blob_bytes(H, I, g) == 32 + 2 * O.q4_bytes(I, H, g) + O.q4_bytes(H, I, g)
    go, uo, do = lp.blob_offsets(H, I, g)
    assert (go, uo, do) == (32, 32 + O.q4_bytes(I, H, g), 32 + 2 * O.q4_bytes(I, H, g))
    b = lp.synth_blob(H, I, g, 1, 2, 3)
    hdr = b[:32].view(np.uint32)
    assert list(hdr) == [64, 128, 64, 128, 128, 64, 64, 0]  # lib.rs:276-281
    # config-1 shape (Qwen3-30B-A3B, H 2048, I 768, group 32): 2,654,240 B per blob
    assert lp.blob_bytes(2048, 768, 32) == 2654240
    assert lp.blob_offsets(2048, 768, 32) == (32, 884768, 1769504)


def test_synth_deterministic_and_thread_independent():
    H, I, g = 256, 128, 32
    span = 65536
    a = lp.synth_blobs(6, span, H, I, g, 0, 3, threads=1)
    b = lp.synth_blobs(6, span, H, I, g, 0, 3, threads=4)
    assert np.array_equal(a, b)
    one = lp.synth_blob(H, I, g, 0, 3, 4)
    assert np.array_equal(a[4 * span: 4 * span + one.size], one)
    assert not np.array_equal(lp.synth_blob(H, I, g, 0, 3, 5), one)
    assert np.array_equal(lp.synth_bf16(100, 0.02, 0, 7), lp.synth_bf16(100, 0.02, 0, 7))


def test_synth_distributions():
    # nibbles uniform 0..15; f16 scales |N(0, 0.02)|/8;
    # router bf16 N(0, 0.02); activations bf16 N(0, 1)
    H, I, g = 2048, 768, 32
    b = lp.synth_blob(H, I, g, 0, 0, 0)
    go, uo, do = lp.blob_offsets(H, I, g)
    ns = I * (H // g)
    sc = b[go: go + 2 * ns].view(np.float16).astype(np.float64)
    assert sc.min() >= 0
    assert abs(sc.mean() - 0.02 * np.sqrt(2 / np.pi) / 8) < 0.02 * 0.02
    nib = b[go + 2 * ns: uo]
    counts = np.bincount(np.concatenate([nib & 15, nib >> 4]), minlength=16)
    assert counts.min() > 0.98 * counts.mean() and counts.max() < 1.02 * counts.mean()
    w = lp.synth_bf16(1 << 16, 0.02, 0, 1)
    wf = (w.astype(np.uint32) << 16).view(np.float32)
    assert abs(wf.std() - 0.02) < 0.001 and abs(wf.mean()) < 0.001
    x = lp.synth_f32_bf16(1 << 16, 1.0, 0, 1)
    assert np.array_equal(x.view(np.uint32) & 0xFFFF, np.zeros_like(x.view(np.uint32)))
    assert abs(x.std() - 1) < 0.02


def test_route_expf_matches_glibc_strided():
    # Every 97th float bit pattern (44 million inputs) against libm expf.
    n = (1 << 32) // 97
    for start in range(0, n, 1 << 22):
        cnt = min(1 << 22, n - start)
        mine = lp.route_expf_sweep(start * 97, 97, cnt)
        ref = O.expf_sweep(start * 97, 97, cnt)
        same = (mine.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(mine) & np.isnan(ref))
        assert same.all(), hex(start * 97 + 97 * int(np.argmin(same)))


@pytest.mark.slow
def test_route_expf_matches_glibc_exhaustive():
    chunk = 1 << 24
    for first in range(0, 1 << 32, chunk):
        mine = lp.route_expf_sweep(first, 1, chunk)
        ref = O.expf_sweep(first, 1, chunk)
        same = (mine.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(mine) & np.isnan(ref))
        assert same.all(), hex(first + int(np.argmin(same)))


def test_layer_desc_layout_matches_header(tmp_path):
    fields = [f[0] for f in lp.LayerDesc._fields_]
    src = tmp_path / "off.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "llmpager_hip.h"\nint main(){'
                   + "".join(f'printf("%zu\\n", offsetof(lp_moe_layer_desc, {f}));' for f in fields)
                   + 'printf("%zu\\n", sizeof(lp_moe_layer_desc));'
                   + "".join(f'printf("%zu\\n", offsetof(lp_moe_ws_layout, {f[0]}));'
                             for f in lp.WsLayout._fields_)
                   + "return 0;}\n")
    exe = tmp_path / "off"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True).stdout.split()]
    want = [getattr(lp.LayerDesc, f).offset for f in fields] + [C.sizeof(lp.LayerDesc)]
    want += [getattr(lp.WsLayout, f[0]).offset for f in lp.WsLayout._fields_]
    assert out == want


def test_ws_layout_alignment_and_size():
    d = lp.LayerDesc(hidden=2048, inter=768, experts=128, top_k=8, group=32)
    for T in (1, 8, 32, 2048):
        lay = lp.ws_layout(d, T)
        offs = [getattr(lay, f[0]) for f in lp.WsLayout._fields_[:-1]]
        assert all(o % 256 == 0 for o in offs)
        assert offs == sorted(offs)
        assert lay.total >= lay.y + T * 8 * 2048 * 4
        # the digit images of x fill their part; the bf16 images only exist
        # for the prefill GEMM (T = 2048 here)
        assert lay.sh_et - lay.xd >= T * lp.dimage_bytes(2048) > lay.sh_et - lay.xd - 256
        assert (lay.xd - lay.xf > 0) == (T == 2048)


def test_workspace_check_rejects_undersized_workspaces():
    """lp_moe_workspace_check, the pre-launch check of every MoE entry point
    that takes a workspace: null, misaligned and short workspaces are refused
    (a short one would be written past its end by the kernels), for one layer
    and for a stack sized by its largest layer."""
    d = lp.LayerDesc(hidden=2048, inter=768, experts=128, top_k=8, group=32, router_w=1 << 20,
                     slot_table=2 << 20, arena_base=1 << 30, slot_span=2658304,
                     gate_off=32, up_off=884768, down_off=1769504)
    for T in (1, 8, 32, 2048):
        need = lp.ws_layout(d, T).total
        ws = 1 << 32
        assert lp.workspace_check([d], T, ws, need) == 0
        assert lp.workspace_check([d], T, ws, need + 4096) == 0
        assert lp.workspace_check([d], T, ws, need - 1) == -1
        assert "needs %d" % need in lp.lib().lp_last_error().decode()
        assert lp.workspace_check([d], T, ws, 0) == -1
        assert lp.workspace_check([d], T, 0, need) == -1
        assert lp.workspace_check([d], T, ws + 16, need) == -2
    # a stack: the largest layer decides; the failing layer is named
    big = lp.LayerDesc(**{f: getattr(d, f) for f, _ in lp.LayerDesc._fields_})
    big.inter = 1536
    big.up_off, big.down_off = lp.blob_offsets(2048, 1536, 32)[1:]
    T = 32
    need = max(lp.ws_layout(x, T).total for x in (d, big))
    assert need > lp.ws_layout(d, T).total
    assert lp.workspace_check([d, big], T, 1 << 32, need) == 0
    assert lp.workspace_check([d, big], T, 1 << 32, lp.ws_layout(d, T).total) == -1
    assert lp.lib().lp_last_error().decode().startswith("layer 1:")
    # a bad descriptor is refused before the size is looked at
    bad = lp.LayerDesc(**{f: getattr(d, f) for f, _ in lp.LayerDesc._fields_})
    bad.top_k = 0
    assert lp.workspace_check([d, bad], T, 1 << 32, 1 << 40) == -2
    # the Python wrappers take the size from an allocation, or refuse
    with pytest.raises(TypeError):
        lp._ws_bytes(1 << 32, None)
    assert lp._ws_bytes(lp.DevPtr(1 << 32, 4096), None) == 4096


def _c_decl_args(text):
    """{name: argument count} of the header's function declarations."""
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(lp_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def _rs_decl_args(text):
    out = {}
    for m in re.finditer(r"pub fn (lp_[a-z0-9_]+)\((.*?)\)\s*(->[^;]*)?;", text, flags=re.S):
        args = [a for a in m.group(2).split(",") if a.strip()]
        out[m.group(1)] = len(args)
    return out


def _c_struct_fields(text, name):
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, flags=re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    fields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        names = decl.split(None, 1)[1] if not decl.startswith("const ") else decl.split(None, 2)[2]
        fields += [re.sub(r"[\s*]|\[.*\]", "", n) for n in names.split(",")]
    return fields


def test_rust_bindings_follow_the_header():
    """rust/llmpager-hip/src/ffi.rs declares only functions the header
    declares, and its repr(C) structs list the header's fields in order."""
    rs = open(os.path.join(ROOT, "rust", "llmpager-hip", "src", "ffi.rs")).read()
    hdr = open(HEADER).read()
    fns = set(re.findall(r"pub fn (lp_[a-z0-9_]+)\(", rs))
    assert len(fns) > 80
    assert not fns - set(declared_functions())
    # and each with the header's number of arguments
    c_args, rs_args = _c_decl_args(hdr), _rs_decl_args(rs)
    assert set(rs_args) == fns
    assert {n: rs_args[n] for n in fns} == {n: c_args[n] for n in fns}
    for st in ("lp_moe_layer_desc", "lp_moe_ws_layout", "lp_pager_config", "lp_pager_metrics", "lp_expert_handle"):
        body = re.search(r"pub struct %s \{(.*?)\n\}" % st, rs, flags=re.S).group(1)
        rs_fields = re.findall(r"pub ([a-z0-9_]+):", body)
        assert rs_fields == _c_struct_fields(hdr, st), st
