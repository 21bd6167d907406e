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

// Global-address-space views: loads through these compile to global_load_*
// (tracked by vmcnt only), not flat_load_*, so many can be in flight at once.
#define LP_GLOBAL __attribute__((address_space(1)))

template <typename T>
__device__ __forceinline__ const LP_GLOBAL T* gptr(uint64_t a) {
    return reinterpret_cast<const LP_GLOBAL T*>(a);
}

template <typename T>
__device__ __forceinline__ LP_GLOBAL T* gptr_w(uint64_t a) {
    return reinterpret_cast<LP_GLOBAL T*>(a);
}

// ---------------------------------------------------------------------------
// The grouped q4 tile.
//
// One wave computes, for a 16-row tile of a q4 region [rows, cols] and for
// pairs of tokens, y[t][row] = sum_g s[row, g >> rs] * sum_{c in sub-group g}
// (q[row, c] - 8) * x[t][c] in fp32.  Sub-groups are 32 columns; one f16
// scale covers 2^rs sub-groups (rs = log2(group / 32)).
//
// MFMA v_mfma_f32_16x16x32_bf16 (C[m][n] += sum_k A[m][k] B[k][n]):
//   B (weights): lane l = (n = l % 16, kb = l / 16).  At step c the four
//     lanes of row n load sub-groups 4c..4c+3 (64 contiguous bytes of the row,
//     16 per lane); MFMA d (0..3) takes the d-th 32-bit word of each load.
//   A (activations): row m = 4*slot + th, th = 2*token + part, part 0 =
//     bf16(x), part 1 = bf16(x - bf16(x)).  Element (m, k = 8*kbA + i) is
//     non-zero only when slot == kbA, so the 16 MFMA output rows keep four
//     sub-groups x four (token, part) apart.
//   C: lane l holds C[4*(l/16) + i][l % 16]: its own sub-group (slot = kb),
//     th = i.  With n = q + 8 the stored nibble, the weight operand is
//     128 + n, so sum_k (128 + n_k) x_k = sum_k (n_k - 8) x_k + 136 sum_k x_k;
//     the accumulator is therefore seeded with -136 * sum_k x_k of the part.
// Products of bf16 values are exact in fp32 and x = part0 + part1 to 16
// significant bits, so the only roundings are the fp32 accumulations.
//
// Activation fragments live in LDS, per token pair p:
//   frag[p][th][g][d] : uint4 (8 bf16 in element order i), th 0..3
//   off [p][g][th]    : float, -136 * sum of the th part over sub-group g
// ---------------------------------------------------------------------------

struct Frags {
    uint4* frag;   // [pairs][4][ng][4]
    float* off;    // [pairs][ng][4]
    int ng;        // sub-groups (cols / 32)
};

__device__ __forceinline__ size_t frag_pair_bytes(int ng) { return (size_t)ng * lpk::kFragBytesPerSubgroup; }

__device__ __forceinline__ Frags frags_at(uint8_t* base, int ng, int pairs) {
    Frags F;
    F.frag = reinterpret_cast<uint4*>(base);
    F.off = reinterpret_cast<float*>(base + (size_t)pairs * ng * 256);
    F.ng = ng;
    return F;
}

// Stage ntok activation rows into fragment pairs 0 .. ceil(ntok/2)-1.
// row_of(t) returns the f32 row of token t.  Work units (token, sub-group)
// are spread over the `nthreads` participating threads (tid < nthreads); a
// missing second token of the last pair is written as zeros.
template <typename RowOf>
__device__ inline void stage_rows(const Frags& F, int ntok, RowOf row_of, int tid, int nthreads) {
    const int units = ((ntok + 1) & ~1) * F.ng;
    for (int u = tid; u < units; u += nthreads) {
        const int t = u / F.ng;
        const int g = u - t * F.ng;
        const int pair = t >> 1, tk = t & 1;
        const LP_GLOBAL float4* p =
            t < ntok ? gptr<float4>(reinterpret_cast<uint64_t>(row_of(t) + (size_t)g * 32)) : nullptr;
        uint4* fr = F.frag + (size_t)pair * 4 * F.ng * 4;
        float shi = 0.0f, slo = 0.0f;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            // columns 8d .. 8d+7; fragment element i holds column frag_col(d, i),
            // so 32-bit word w pairs columns 8d + w and 8d + w + 4
            float v[8];
            if (p) {
                const float4 f0 = p[2 * d], f1 = p[2 * d + 1];
                v[0] = f0.x; v[1] = f0.y; v[2] = f0.z; v[3] = f0.w;
                v[4] = f1.x; v[5] = f1.y; v[6] = f1.z; v[7] = f1.w;
            } else {
#pragma unroll
                for (int q = 0; q < 8; ++q) v[q] = 0.0f;
            }
            uint32_t hi[8], lo[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                hi[q] = f32_to_bf16_rne(v[q]);
                lo[q] = f32_to_bf16_rne(v[q] - bf16_to_f32(hi[q]));
                shi += bf16_to_f32(hi[q]);
                slo += bf16_to_f32(lo[q]);
            }
            const uint4 a = make_uint4(hi[0] | (hi[4] << 16), hi[1] | (hi[5] << 16),
                                       hi[2] | (hi[6] << 16), hi[3] | (hi[7] << 16));
            const uint4 b = make_uint4(lo[0] | (lo[4] << 16), lo[1] | (lo[5] << 16),
                                       lo[2] | (lo[6] << 16), lo[3] | (lo[7] << 16));
            fr[((size_t)(2 * tk + 0) * F.ng + g) * 4 + d] = a;
            fr[((size_t)(2 * tk + 1) * F.ng + g) * 4 + d] = b;
        }
        float* of = F.off + ((size_t)pair * F.ng + g) * 4;
        of[2 * tk + 0] = -136.0f * shi;
        of[2 * tk + 1] = -136.0f * slo;
    }
}

__device__ __forceinline__ int tile_steps(int cols) { return ((cols >> 5) + 3) >> 2; }

// Raw weight registers for steps [c0, c0 + NS) of one 16-row tile.
template <int NS>
struct WRegs {
    uint4 w[NS];
    uint32_t s[NS];  // f16 bits of the lane's sub-group scale
};

// Issue the tile's loads: lane (n, kb) loads sub-group 4c + kb of row n0 + n.
template <int NS>
__device__ __forceinline__ void wload(WRegs<NS>& R, uint64_t region, int rows, int cols, int rs,
                                      int n0, int c0) {
    const int lane = lane_id();
    const int n = lane & 15, kb = lane >> 4;
    const int ng = cols >> 5;
    const int row = n0 + n;
    const int gpr = ng >> rs;
    const bool rowok = row < rows;
    const LP_GLOBAL uint4* data = gptr<uint4>(region + (uint64_t)rows * gpr * 2) +
                                  (size_t)row * (cols >> 5);
    const LP_GLOBAL uint16_t* sc = gptr<uint16_t>(region) + (size_t)row * gpr;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const int g = 4 * (c0 + j) + kb;
        if (rowok && g < ng) {
            R.w[j] = data[g];
            R.s[j] = sc[g >> rs];
        } else {
            R.w[j] = make_uint4(0, 0, 0, 0);
            R.s[j] = 0u;
        }
    }
}

// MFMAs for steps [c0, c0 + NS) against `pairs` staged token pairs
// (pairs <= PMAX), accumulating acc[p][0..1] (tokens 2p, 2p+1) per lane.
template <int NS, int PMAX>
__device__ __forceinline__ void wmma(const WRegs<NS>& R, const Frags& F, int cols, int c0, int pairs,
                                     float (&acc)[PMAX][2]) {
    const int lane = lane_id();
    const int kb = lane >> 4;
    const int m = lane & 15;
    const int ng = cols >> 5;
    const int S = tile_steps(cols);
    const bool aact = (m >> 2) == kb;   // A lane (m, kb) is live when its slot m/4 == kb
    const int th = m & 3;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const int c = c0 + j;
        if (c >= S) break;
        const int g = 4 * c + kb;
        const bool gok = g < ng;
        const int gs = gok ? g : 0;
        const float s = f16_bits_to_f32(R.s[j]);
        bf16x8_t bv[4];
        bv[0] = q4_word_to_bf16x8(R.w[j].x);
        bv[1] = q4_word_to_bf16x8(R.w[j].y);
        bv[2] = q4_word_to_bf16x8(R.w[j].z);
        bv[3] = q4_word_to_bf16x8(R.w[j].w);
#pragma unroll
        for (int p = 0; p < PMAX; ++p) {
            if (p < pairs) {
                const float4 o = *reinterpret_cast<const float4*>(F.off + ((size_t)p * ng + gs) * 4);
                f32x4_t cacc;
                cacc[0] = o.x;
                cacc[1] = o.y;
                cacc[2] = o.z;
                cacc[3] = o.w;
                const uint4* fr = F.frag + (((size_t)p * 4 + th) * ng + gs) * 4;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    uint4 a = make_uint4(0, 0, 0, 0);
                    if (aact && gok) a = fr[d];
                    cacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8_t, a), bv[d], cacc, 0, 0, 0);
                }
                acc[p][0] = __builtin_fmaf(s, cacc[0] + cacc[1], acc[p][0]);
                acc[p][1] = __builtin_fmaf(s, cacc[2] + cacc[3], acc[p][1]);
            }
        }
    }
}

// Sum the four kb partials of row n: afterwards every lane (n, *) holds the row.
__device__ __forceinline__ float tile_reduce(float v) {
    v += shfl_xor(v, 16);
    v += shfl_xor(v, 32);
    return v;
}

__device__ __forceinline__ int ilog2_pow2(int v) { return 31 - __builtin_clz(v); }

}  // namespace lp
