"""GPU parity of the 1:1 launchers (kernels.rs hot-path methods) against the
CPU oracle.  Tolerances are the reference's own (gemv_bench.rs:61-71,
kernels_bench.rs:136-161) unless the build's order makes the result exact."""
import numpy as np
import pytest

import llmpager_amd as lp
import _oracle as O
from _gpu import align, rel_l2, worst_rel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,cols,group,experts,x_stride", [
    (768, 2048, 32, 8, 0),      # gate/up, config 1
    (2048, 768, 32, 8, 768),    # down, config 1 (x per expert)
    (768, 2048, 64, 8, 0),      # the reference's own q4g64 packs
    (64, 128, 64, 2, 128),      # write_test_checkpoint shape (lib.rs:341-423)
    (100, 96, 32, 3, 96),       # ragged rows, unaligned nibble rows: VALU path
    (100, 128, 32, 3, 128),     # ragged rows on the MFMA tile
    (48, 96, 32, 2, 96),        # a partial last sub-group step (cols/32 = 3)
    (40, 64, 8, 2, 64),         # group 8: generic VALU path
])
def test_q4_gemv_batch(cuda, rows, cols, group, experts, x_stride):
    rng = np.random.default_rng(rows * 7 + cols)
    H, I = (cols, rows) if rows <= cols else (rows, cols)
    qb = lp.q4_bytes(rows, cols, group)
    span = align(qb + 64)
    host = np.zeros(experts * span, np.uint8)
    regions = []
    for e in range(experts):
        w = rng.standard_normal(rows * cols).astype(np.float32) * 0.05
        buf, _ = O.q4_quantize(w, rows, cols, group)
        host[e * span + 32: e * span + 32 + qb] = buf
        regions.append(buf)
    nx = cols if x_stride == 0 else x_stride * experts
    x = rng.standard_normal(nx).astype(np.float32)
    arena = cuda.upload(host)
    ptrs = np.array([arena + e * span for e in range(experts)], np.uint64)
    d_ptrs = cuda.upload(ptrs)
    d_x = cuda.upload(x)
    d_y = cuda.alloc_device(experts * rows * 4)
    k = lp.Kernels(cuda)
    k.q4g64_gemv_batch(d_ptrs, 32, d_x, x_stride, d_y, rows, cols, group, experts)
    y = cuda.download(d_y, (experts, rows), np.float32)
    for e in range(experts):
        want = O.q4_gemv(regions[e], x[e * x_stride: e * x_stride + cols], rows, cols, group)
        assert worst_rel(y[e], want) <= 1e-3
        # the MFMA path carries x as 16-bit fixed point per 32 columns
        # (within 2^-16 of each sub-group's largest magnitude): rel-L2 ~2e-5
        assert rel_l2(y[e], want) <= 1e-4
    # single-matrix form
    k.q4g64_gemv(arena + 32, d_x, d_y, rows, cols, group)
    y1 = cuda.download(d_y, (rows,), np.float32)
    want = O.q4_gemv(regions[0], x[:cols], rows, cols, group)
    assert rel_l2(y1, want) <= 1e-4
    for p in (arena, d_ptrs, d_x, d_y):
        cuda.free_device(p)


@pytest.mark.parametrize("rows,cols", [(128, 2048), (64, 128), (7, 13), (4096, 4096)])
def test_bf16_gemv(cuda, rows, cols):
    rng = np.random.default_rng(rows + cols)
    w = lp.synth_bf16(rows * cols, 0.02, 5, rows)
    x = rng.standard_normal(cols).astype(np.float32)
    d_w, d_x = cuda.upload(w), cuda.upload(x)
    d_y = cuda.alloc_device(rows * 4)
    lp.Kernels(cuda).bf16_gemv(d_w, d_x, d_y, rows, cols)
    y = cuda.download(d_y, (rows,), np.float32)
    want = O.bf16_gemv(w, x, rows, cols)
    assert worst_rel(y, want) <= 1e-4          # kernels_bench.rs:148-149
    if cols % 8 == 0:
        # the canonical router order: bit-identical to the oracle's restatement
        canon = np.array([O.router_logits(w[r * cols:(r + 1) * cols], x, 1, cols)[0]
                          for r in range(rows)], np.float32)
        assert np.array_equal(y.view(np.uint32), canon.view(np.uint32))
    for p in (d_w, d_x, d_y):
        cuda.free_device(p)


def test_silu_add_reduce(cuda):
    rng = np.random.default_rng(3)
    n = 1000
    a = rng.standard_normal(n).astype(np.float32) * 3
    b = rng.standard_normal(n).astype(np.float32)
    k = lp.Kernels(cuda)
    da, db, dout = cuda.upload(a), cuda.upload(b), cuda.alloc_device(n * 4)
    k.silu_mul(da, db, dout, n)
    assert worst_rel(cuda.download(dout, (n,), np.float32), O.silu_mul(a, b)) <= 1e-4
    k.add(da, db, n)
    assert worst_rel(cuda.download(da, (n,), np.float32), O.add(a, b)) <= 1e-5
    # moe_reduce: same fused order as the oracle restatement -> bit-exact
    E, H = 8, 2048
    eo = rng.standard_normal((E, H)).astype(np.float32)
    wt = rng.random(E).astype(np.float32)
    h = rng.standard_normal(H).astype(np.float32)
    deo, dwt, dh = cuda.upload(eo), cuda.upload(wt), cuda.upload(h)
    k.moe_reduce(deo, dwt, dh, E, H)
    got = cuda.download(dh, (H,), np.float32)
    assert np.array_equal(got, O.moe_reduce(eo, wt, h))
    for p in (da, db, dout, deo, dwt, dh):
        cuda.free_device(p)


def _device_expf(cuda, first, stride, n):
    out = cuda.alloc_device(n * 4)
    assert lp.lib().lp_route_expf_device(cuda.ctx, first, stride, n, out, None) == 0
    got = cuda.download(out, (n,), np.float32)
    cuda.free_device(out)
    return got


@pytest.mark.parametrize("first,stride,n", [
    (0, 9973, (1 << 32) // 9973),     # a spread over every float
    (0x42b00000 - 2048, 1, 4096),     # around 88.0 (the special-case cut)
    (0x42b17218 - 2048, 1, 4096),     # around the overflow threshold
    (0xc2cff1b4 - 2048, 1, 4096),     # around the underflow threshold
    (0x7f800000 - 2048, 1, 4096),     # largest finite, +inf, NaNs
    (0xff800000 - 2048, 1, 4096),     # most negative finite, -inf, NaNs
    (0x00000000, 1, 8192),            # +0 and denormals
    (0x80000000, 1, 8192),            # -0 and negative denormals
    (0x3f800000 - 4096, 1, 8192),     # around 1.0
])
def test_device_expf_matches_glibc(cuda, first, stride, n):
    # The routing kernels' expf (glibc's method, table in registers) against
    # this host's glibc expf, bit for bit.
    got = _device_expf(cuda, first, stride, n)
    want = O.expf_sweep(first, stride, n)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), hex((first + stride * int(np.argmin(same))) & 0xffffffff)
