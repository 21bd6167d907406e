// gfx950 kernels behind the 1:1 launchers that replace the hot-path methods of
// the reference's `Kernels` (crates/llmpager-cuda/src/kernels.rs).  Same
// semantics and argument meaning; the arithmetic is this build's own.
#include "lp_device.h"

using namespace lp;
using namespace lpk;

// ---------------------------------------------------------------------------
// q4 GEMV, batched over experts (kernels.rs:102-127, q4g64.cu:19-81 semantics):
//   y[e*rows + r] = sum_g s[r, g] * sum_{c in g} (q[r, c] - 8) * x_e[c],
//   x_e = x + e*x_stride, region = blobs[e] + region_off.
// MFMA path: grid (workgroups per expert, experts); the workgroup stages x_e
// once into an LDS fragment pair, then each wave walks 16-row tiles.
// Requires group = 32 * 2^r, 16-byte aligned nibble rows and x (host checks).
// Dynamic LDS: lpk::frag_lds_bytes(cols, 1).
// ---------------------------------------------------------------------------
template <int RS>
__device__ __forceinline__ void q4_gemv_tiles(const Q4GemvBatchArgs& a, const Frags& F, uint64_t region,
                                              float* y) {
    const int wave = threadIdx.x >> 6;
    const int wpb = blockDim.x >> 6;
    const int lane = lane_id();
    const int tiles = (a.rows + kTileRows - 1) / kTileRows;
    const int S = tile_steps(a.cols);
    for (int tile = blockIdx.x * wpb + wave; tile < tiles; tile += gridDim.x * wpb) {
        const int n0 = tile * kTileRows;
        const WTile<RS> T = wtile<RS>(region, a.rows, a.cols, n0);
        float acc[1][1][2] = {{{0.0f, 0.0f}}};
        WRegs<kGemvChunk> R[1];
        wload(R[0], T, 0);
#pragma nounroll
        for (int c0 = 0;;) {
            const ABase B[1] = {abase(F, 0, c0)};
            wmma(R, B, S - c0, 1, acc);
            c0 += kGemvChunk;
            if (c0 >= S) break;
            wload(R[0], T, c0);
        }
        const float v = tile_reduce(acc[0][0][0]);
        const int row = n0 + (lane & 15);
        if (lane < 16 && row < a.rows) y[row] = v;
    }
}

extern "C" __global__ void __launch_bounds__(256) lp_q4_gemv_mfma(const Q4GemvBatchArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int e = blockIdx.y;
    const uint64_t region = a.blobs ? gptr<uint64_t>(a.blobs)[e] + a.region_off : a.region_off;
    const float* x = reinterpret_cast<const float*>(a.x) + (size_t)e * a.x_stride;
    float* y = reinterpret_cast<float*>(a.y) + (size_t)e * a.rows;
    const Frags F = frags_at(lds, a.cols);
    zero_block(F, threadIdx.x, blockDim.x);
    stage_rows(F, 1, [&](int) { return x; }, threadIdx.x, blockDim.x);
    __syncthreads();
    switch (ilog2_pow2(a.group >> 5)) {
        case 0: q4_gemv_tiles<0>(a, F, region, y); break;
        case 1: q4_gemv_tiles<1>(a, F, region, y); break;
        default: q4_gemv_tiles<2>(a, F, region, y); break;
    }
}

// Generic VALU form for any group % 8 == 0 (and unaligned operands): one wave
// per row, each lane owns whole groups, fp32 FMAs on exactly dequantised
// values, butterfly reduction.
extern "C" __global__ void __launch_bounds__(256) lp_q4_gemv_valu(const Q4GemvBatchArgs a) {
    const int e = blockIdx.y;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = lane_id();
    if (row >= a.rows) return;
    const uint64_t blob = a.blobs ? reinterpret_cast<const uint64_t*>(a.blobs)[e] : a.region_off;
    const uint8_t* region = reinterpret_cast<const uint8_t*>(a.blobs ? blob + a.region_off : blob);
    const float* x = reinterpret_cast<const float*>(a.x) + (size_t)e * a.x_stride;
    const int gpr = a.cols / a.group;
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(region) + (size_t)row * gpr;
    const uint8_t* data = region + (size_t)a.rows * gpr * 2 + (size_t)row * (a.cols >> 1);
    float acc = 0.0f;
    for (int g = lane; g < gpr; g += 64) {
        const float s = f16_bits_to_f32(sc[g]);
        const uint8_t* d = data + (size_t)g * (a.group >> 1);
        const float* xg = x + (size_t)g * a.group;
        float sum = 0.0f;
        for (int i = 0; i < (a.group >> 1); ++i) {
            const uint32_t b = d[i];
            sum = __builtin_fmaf((float)((int)(b & 15u) - 8), xg[2 * i], sum);
            sum = __builtin_fmaf((float)((int)(b >> 4) - 8), xg[2 * i + 1], sum);
        }
        acc = __builtin_fmaf(s, sum, acc);
    }
    for (int o = 32; o >= 1; o >>= 1) acc += shfl_xor(acc, o);
    if (lane == 0) reinterpret_cast<float*>(a.y)[(size_t)e * a.rows + row] = acc;
}

// out[i] += sum_e wts[e] * eouts[e, i]   (q4g64.cu:84-99: pick order, then one add)
extern "C" __global__ void __launch_bounds__(256) lp_moe_reduce(const MoeReduceArgs a) {
    const float* eo = reinterpret_cast<const float*>(a.eouts);
    const float* w = reinterpret_cast<const float*>(a.wts);
    float* out = reinterpret_cast<float*>(a.out);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += gridDim.x * blockDim.x) {
        float acc = 0.0f;
        for (int e = 0; e < a.experts; ++e) acc = __builtin_fmaf(w[e], eo[(size_t)e * a.n + i], acc);
        out[i] += acc;
    }
}

// out = g / (1 + exp(-g)) * u   (decode.cu:117-128)
extern "C" __global__ void __launch_bounds__(256) lp_silu_mul(const SiluMulArgs a) {
    const float* g = reinterpret_cast<const float*>(a.gate);
    const float* u = reinterpret_cast<const float*>(a.up);
    float* out = reinterpret_cast<float*>(a.out);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += gridDim.x * blockDim.x) {
        const float v = g[i];
        out[i] = v / (1.0f + expf(-v)) * u[i];
    }
}

// a += b   (decode.cu:131-140)
extern "C" __global__ void __launch_bounds__(256) lp_add(const AddArgs a) {
    float* pa = reinterpret_cast<float*>(a.a);
    const float* pb = reinterpret_cast<const float*>(a.b);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += gridDim.x * blockDim.x)
        pa[i] += pb[i];
}

// y = W x, W bf16 [rows, cols]   (decode.cu:80-114 semantics).  One wave per
// row.  For cols % 8 == 0 this is exactly the router's canonical order: lane l
// takes 8-column chunks l, l+64, ... with fused multiply-adds, then a
// butterfly over the 64 lanes.  Other widths add a scalar tail per lane.
extern "C" __global__ void __launch_bounds__(256) lp_bf16_gemv(const Bf16GemvArgs a) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = lane_id();
    if (row >= a.rows) return;
    const uint16_t* w = reinterpret_cast<const uint16_t*>(a.w) + (size_t)row * a.cols;
    const float* x = reinterpret_cast<const float*>(a.x);
    float acc = 0.0f;
    const int chunks = a.cols >> 3;
    const bool vec = (a.cols & 7) == 0;
    if (vec) {
        for (int ch = lane; ch < chunks; ch += 64) {
            const uint4 wv = *reinterpret_cast<const uint4*>(w + ch * 8);
            const float4 xa = *reinterpret_cast<const float4*>(x + ch * 8);
            const float4 xb = *reinterpret_cast<const float4*>(x + ch * 8 + 4);
            acc = __builtin_fmaf(bf16_to_f32(wv.x & 0xffffu), xa.x, acc);
            acc = __builtin_fmaf(bf16_to_f32(wv.x >> 16), xa.y, acc);
            acc = __builtin_fmaf(bf16_to_f32(wv.y & 0xffffu), xa.z, acc);
            acc = __builtin_fmaf(bf16_to_f32(wv.y >> 16), xa.w, acc);
            acc = __builtin_fmaf(bf16_to_f32(wv.z & 0xffffu), xb.x, acc);
            acc = __builtin_fmaf(bf16_to_f32(wv.z >> 16), xb.y, acc);
            acc = __builtin_fmaf(bf16_to_f32(wv.w & 0xffffu), xb.z, acc);
            acc = __builtin_fmaf(bf16_to_f32(wv.w >> 16), xb.w, acc);
        }
    } else {
        for (int c = lane; c < a.cols; c += 64) acc = __builtin_fmaf(bf16_to_f32(w[c]), x[c], acc);
    }
    for (int o = 32; o >= 1; o >>= 1) acc += shfl_xor(acc, o);
    if (lane == 0) reinterpret_cast<float*>(a.y)[row] = acc;
}

// expf over float bit patterns, the way routing evaluates it on the device
// (expf_glibc_wave: table in registers, whole waves): out[i] =
// expf(bits(first + i * stride)), i < n.  For parity checks against glibc.
extern "C" __global__ void __launch_bounds__(256) lp_expf_wave(const ExpfSweepArgs a) {
    const uint64_t tabv = exp2tab_lane();
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint32_t bits = a.first + (uint32_t)(i * a.stride);
    const float y = expf_glibc_wave(__uint_as_float(bits), tabv);  // every lane, in or out of range
    if (i < a.n) reinterpret_cast<float*>(a.out)[i] = y;
}
