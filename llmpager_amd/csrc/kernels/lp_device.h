// Device helpers shared by the gfx950 kernels: conversions, wave reductions,
// and the q4 x bf16 MFMA tile that every grouped expert projection runs on.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../lp_expf.h"
#include "../lp_kargs.h"

namespace lp {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Round-to-nearest-even f32 -> bf16 bits (inputs are finite).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    uint32_t b = __float_as_uint(f);
    return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63u); }

__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    for (int o = 32; o >= 1; o >>= 1) {
        uint64_t w = __shfl_xor(v, o, 64);
        v = w > v ? w : v;
    }
    return v;
}

// Eight q4 values (one 32-bit word, value p at bits [4p, 4p+4), stored as q+8)
// as eight bf16 of value 128 + (q+8).  0x4300 is bf16 128.0, whose unit in the
// last place is 1, so OR-ing a nibble into the low mantissa bits adds it
// exactly.  Element i = 2v + h of the result holds value p = v + 4h, so the
// activation fragment must be laid out in the same order (see frag_col).
__device__ __forceinline__ bf16x8_t q4_word_to_bf16x8(uint32_t b) {
    u32x4_t t;
    t[0] = (b & 0x000F000Fu) | 0x43004300u;
    t[1] = ((b >> 4) & 0x000F000Fu) | 0x43004300u;
    t[2] = ((b >> 8) & 0x000F000Fu) | 0x43004300u;
    t[3] = ((b >> 12) & 0x000F000Fu) | 0x43004300u;
    return __builtin_bit_cast(bf16x8_t, t);
}

// Column (within a 32-column sub-group) of fragment element i of chunk d.
__device__ __forceinline__ int frag_col(int d, int i) { return 8 * d + (i >> 1) + 4 * (i & 1); }

// ---------------------------------------------------------------------------
// The grouped q4 tile.
//
// One wave computes, for a 16-row tile of a q4 region [rows, cols] and for up
// to two tokens, y[t][row] = sum_g s[row, g/R] * sum_{c in sub-group g}
// (q[row, c] - 8) * x[t][c] in fp32, where sub-groups are 32 columns and
// R = group / 32 (one scale covers R sub-groups).
//
// MFMA v_mfma_f32_16x16x32_bf16 (C[m][n] += sum_k A[m][k] B[k][n]):
//   B (weights): lane l = (n = l % 16, kb = l / 16) holds 8 values of row n;
//     lane kb owns the contiguous sub-group range [kb*S, kb*S + S) with
//     S = ceil(cols/32 / 4), and at step c loads its whole 16-byte sub-group
//     kb*S + c.  MFMA d (0..3) takes the d-th 32-bit word of that load.
//   A (activations): row m = 4*slot + th, slot = kb of the B lanes it pairs
//     with, th = 2*token + part, part 0 = bf16(x), part 1 = bf16(x - bf16(x)).
//     Element (m, k = 8*kbA + i) is non-zero only when slot == kbA, so the
//     16 MFMA output rows keep four sub-groups x four (token, part) apart.
//   C: lane l holds C[4*(l/16) + i][l % 16]: its own sub-group (slot = kb),
//     th = i.  With n = q + 8 the stored nibble, the weight operand is
//     128 + n, so sum_k (128 + n_k) x_k = sum_k (n_k - 8) x_k + 136 sum_k x_k;
//     the accumulator is therefore seeded with -136 * sum_k x_k of the part.
// Products of bf16 values are exact in fp32 and x = part0 + part1 to 16
// significant bits, so the only roundings are the fp32 accumulations.
//
// Activation fragments live in LDS, per wave:
//   frag[th][g][d] : uint4 (8 bf16 in element order i), th 0..3, g < NG
//   off [g][th]    : float, -136 * sum of the th part over sub-group g
// ---------------------------------------------------------------------------

struct FragLds {
    uint4* frag;   // [4][ng][4]
    float* off;    // [ng][4]
    int ng;        // sub-groups (cols / 32)
};

__device__ __forceinline__ size_t frag_lds_bytes(int ng) { return (size_t)ng * (4 * 4 * 16 + 16); }

// Stage up to two activation rows (f32) into the per-wave fragment layout.
// x0 / x1 may be null (token absent: its rows become zero).  All 64 lanes
// participate; lane L handles sub-groups L, L + 64, ...
__device__ inline void stage_frags(const FragLds& F, const float* x0, const float* x1) {
    const int lane = lane_id();
    for (int g = lane; g < F.ng; g += 64) {
        for (int t = 0; t < 2; ++t) {
            const float* x = t == 0 ? x0 : x1;
            float v[32];
            if (x) {
                const float4* p = reinterpret_cast<const float4*>(x + (size_t)g * 32);
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    float4 f = p[q];
                    v[4 * q + 0] = f.x;
                    v[4 * q + 1] = f.y;
                    v[4 * q + 2] = f.z;
                    v[4 * q + 3] = f.w;
                }
            } else {
#pragma unroll
                for (int q = 0; q < 32; ++q) v[q] = 0.0f;
            }
            uint32_t hi[32], lo[32];
            float shi = 0.0f, slo = 0.0f;
#pragma unroll
            for (int q = 0; q < 32; ++q) {
                hi[q] = f32_to_bf16_rne(v[q]);
                float r = v[q] - bf16_to_f32(hi[q]);
                lo[q] = f32_to_bf16_rne(r);
                shi += bf16_to_f32(hi[q]);
                slo += bf16_to_f32(lo[q]);
            }
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                uint4 a, b;
                uint32_t* pa = reinterpret_cast<uint32_t*>(&a);
                uint32_t* pb = reinterpret_cast<uint32_t*>(&b);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const int c0 = frag_col(d, 2 * w), c1 = frag_col(d, 2 * w + 1);
                    pa[w] = hi[c0] | (hi[c1] << 16);
                    pb[w] = lo[c0] | (lo[c1] << 16);
                }
                F.frag[((size_t)(2 * t + 0) * F.ng + g) * 4 + d] = a;
                F.frag[((size_t)(2 * t + 1) * F.ng + g) * 4 + d] = b;
            }
            F.off[g * 4 + 2 * t + 0] = -136.0f * shi;
            F.off[g * 4 + 2 * t + 1] = -136.0f * slo;
        }
    }
}

// Raw weight loads for steps [c0, c0 + NSTEP) of one 16-row tile: lane
// (n, kb) loads sub-group kb*S + c of row n0 + n and its scale, where
// S = ceil(cols/32 / 4) is the number of steps a lane walks for the row.
template <int NSTEP>
struct TileRegs {
    uint4 w[NSTEP];
    float s[NSTEP];
};

__device__ __forceinline__ int tile_steps(int cols) { return ((cols >> 5) + 3) >> 2; }

template <int NSTEP>
__device__ __forceinline__ void tile_load(TileRegs<NSTEP>& R, const uint8_t* region, int rows,
                                          int cols, int group, int n0, int c0) {
    const int lane = lane_id();
    const int n = lane & 15, kb = lane >> 4;
    const int ng = cols >> 5;
    const int S = tile_steps(cols);
    const int row = n0 + n;
    const int rdiv = group >> 5;
    const int gpr = cols / group;
    const bool rowok = row < rows;
    const uint8_t* data = region + (size_t)rows * gpr * 2 + (size_t)row * (cols >> 1);
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(region) + (size_t)row * gpr;
#pragma unroll
    for (int j = 0; j < NSTEP; ++j) {
        const int c = c0 + j;
        const int g = kb * S + c;
        const bool ok = rowok && c < S && g < ng;
        if (ok) {
            R.w[j] = *reinterpret_cast<const uint4*>(data + (size_t)g * 16);
            R.s[j] = f16_bits_to_f32(sc[g / rdiv]);
        } else {
            R.w[j] = make_uint4(0, 0, 0, 0);
            R.s[j] = 0.0f;
        }
    }
}

// MFMAs for steps [c0, c0 + NSTEP) of a loaded tile against the staged
// fragments, accumulated into per-lane partial sums for token 0 and token 1
// (lane (n, kb) covers its own sub-groups only; reduce over kb with
// tile_reduce).
template <int NSTEP>
__device__ __forceinline__ void tile_mma(const TileRegs<NSTEP>& R, const FragLds& F, int cols,
                                         int c0, float& acc0, float& acc1) {
    const int lane = lane_id();
    const int kb = lane >> 4;
    const int m = lane & 15;
    const int ng = cols >> 5;
    const int S = tile_steps(cols);
    // A-operand lane (m, kbA = kb): active when its slot m/4 equals kbA.
    const bool aact = (m >> 2) == kb;
    const int th = m & 3;
#pragma unroll
    for (int j = 0; j < NSTEP; ++j) {
        const int c = c0 + j;
        if (c >= S) break;
        const int g = kb * S + c;
        const bool gok = g < ng;
        const int gs = gok ? g : 0;
        f32x4_t acc;
        const float4 o = *reinterpret_cast<const float4*>(F.off + gs * 4);
        acc[0] = o.x;
        acc[1] = o.y;
        acc[2] = o.z;
        acc[3] = o.w;
        const uint4 wv = R.w[j];
        const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            uint4 a = make_uint4(0, 0, 0, 0);
            if (aact && gok) a = F.frag[((size_t)th * F.ng + gs) * 4 + d];
            const bf16x8_t av = __builtin_bit_cast(bf16x8_t, a);
            const bf16x8_t bv = q4_word_to_bf16x8(wd[d]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
        }
        const float s = R.s[j];
        acc0 = __builtin_fmaf(s, acc[0] + acc[1], acc0);
        acc1 = __builtin_fmaf(s, acc[2] + acc[3], acc1);
    }
}

// Sum the four kb partials of row n: afterwards every lane (n, *) holds the row.
__device__ __forceinline__ float tile_reduce(float v) {
    v += shfl_xor(v, 16);
    v += shfl_xor(v, 32);
    return v;
}

}  // namespace lp
