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

// Wave-wide reduction of a 32-bit value through DPP (gfx9 row shifts and row
// broadcasts, no LDS traffic); every lane gets the result.  ident is the
// identity of op, read where a lane has no source.  Lane i of each row first
// gathers lanes i-3..i of the original value, then i-7..i and i-15..i of the
// running value; row broadcasts fold rows 0+1 into lane 31 and all four rows
// into lane 63.
template <typename Op>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v0, uint32_t ident, Op op) {
    const int id = (int)ident;
    uint32_t v = op(v0, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v0, 0x111, 0xf, 0xf, false));
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v0, 0x112, 0xf, 0xf, false));  // row_shr:2
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v0, 0x113, 0xf, 0xf, false));  // row_shr:3
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x114, 0xf, 0xe, false));   // row_shr:4
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x118, 0xf, 0xc, false));   // row_shr:8
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x142, 0xa, 0xf, false));   // row_bcast:15
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x143, 0xc, 0xf, false));   // row_bcast:31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Inclusive prefix sum over the wave's lanes through DPP (no LDS traffic):
// row shifts by 1, 2, 4 and 8 (Hillis-Steele within each row of 16, lanes
// shifted in from outside the row read 0), then row 0's total broadcast into
// rows 1 and 3 (row_bcast:15) and lane 31's running sum into rows 2 and 3
// (row_bcast:31).  Every lane must take part.
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15 into rows 1, 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31 into rows 2, 3
    return v;
}

// Hand-offs between workgroups of one launch: stores that write through to
// agent scope, loads at agent scope, a count of completed parts and a
// bounded wait for it.
template <typename T>
__device__ __forceinline__ void agent_store(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T agent_load(const T* p) {
    return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One more completed part at *cnt once this workgroup's stores have
// completed (every thread calls it).
__device__ __forceinline__ void signal_count(int* cnt) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) atomicAdd(cnt, 1);
}

// Wait until *cnt reaches target (every thread calls it), polling with
// agent-scope loads.  The counted parts come from workgroups of lower index
// in the same launch, dispatched before this one on its XCD; the wait is
// bounded all the same (spin_max polls of about a microsecond each): one
// that gives up adds one to *err and goes on, so every wave still ends.
__device__ __forceinline__ void wait_count(int* cnt, int target, int* err, int spin_max) {
    if (threadIdx.x == 0) {
        int it = 0;
        while (agent_load(cnt) < target) {
            if (++it >= spin_max) {
                atomicAdd(err, 1);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    return wave_reduce_u32(v, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    return wave_reduce_u32(v, 0xffffffffu, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}

// Eight q4 values (one 32-bit word, value p at bits [4p, 4p+4), stored as q+8)
// as eight bf16 of value 128 + (q+8).  0x4300 is bf16 128.0, whose unit in the
// last place is 1, so OR-ing a nibble into the low mantissa bits adds it
// exactly.  Element i = 2v + h of the result holds value p = v + 4h, so the
// activation fragment must be laid out in the same order (see frag_col).
// v_bitop3_b32 computes (b & mask) | magic in one instruction (truth table
// 0xEA = (S0 & S1) | S2).
__device__ __forceinline__ uint32_t and_or(uint32_t b, uint32_t m, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(b, m, c, 0xEA);
}

__device__ __forceinline__ bf16x8_t q4_word_to_bf16x8(uint32_t b) {
    u32x4_t t;
    t[0] = and_or(b, 0x000F000Fu, 0x43004300u);
    t[1] = and_or(b >> 4, 0x000F000Fu, 0x43004300u);
    t[2] = and_or(b >> 8, 0x000F000Fu, 0x43004300u);
    t[3] = and_or(b >> 12, 0x000F000Fu, 0x43004300u);
    return __builtin_bit_cast(bf16x8_t, t);
}

// Column (within a 32-column sub-group) of fragment element i of chunk d.
__device__ __forceinline__ int frag_col(int d, int i) { return 8 * d + (i >> 1) + 4 * (i & 1); }

// Global-address-space views: loads through these compile to global_load_*
// (tracked by vmcnt only), not flat_load_*, so many can be in flight at once.
#define LP_GLOBAL __attribute__((address_space(1)))

// Word 3 of a raw (stride 0) buffer resource on gfx9-family parts: 32-bit
// data format, no swizzle; out-of-range loads return zero.
constexpr int kBufferWord3 = 0x00020000;

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
// One wave computes, for a 16-row tile of a q4 region [rows, cols] and for P
// pairs of tokens, y[t][row] = sum_g s[row, g >> rs] * sum_{c in sub-group g}
// (q[row, c] - 8) * x[t][c] in fp32.  Sub-groups are 32 columns; one f16
// scale covers 2^rs sub-groups (rs = log2(group / 32)).
//
// Activations are integer digits: per (token, sub-group) the 32 values are
// 16-bit fixed point against their largest magnitude m, xq = rint(x * 32639
// / m) with sigma = m / 32639, written as two int8 digits hi = (xq + 128) >>
// 8 and lo = xq - 256 hi.  The stored nibbles n = q + 8 (0 .. 15) are the
// weight operand as they are, one AND (even columns) or a shift and an AND
// (odd columns) per four.
//
// MFMA v_mfma_i32_16x16x64_i8 (C[m][n] += sum_k A[m][k] B[k][n]):
//   B (weights): lane l = (n = l % 16, kb = l / 16).  At step c the four
//     lanes of row n load sub-groups 4c..4c+3 (64 contiguous bytes of the row,
//     16 per lane: words w0..w3 = columns 0-7, 8-15, 16-23, 24-31); MFMA h
//     (0, 1) takes w & 0x0F0F0F0F and (w >> 4) & 0x0F0F0F0F of words 2h and
//     2h + 1, i.e. byte t of the lane's 16 holds column
//     16h + 8 (t >> 3) + 2 (t & 3) + ((t >> 2) & 1)  (digit_col).
//   A (activations): row m = 4*slot + th, th = 2*token + digit (0 = hi, 1 =
//     lo).  Element (m, k = 16*kbA + t) is non-zero only when slot == kbA, so
//     the 16 output rows keep four sub-groups x four (token, digit) apart.
//     Lanes whose slot is not their kb read a zero block, so every LDS read
//     is unconditional.
//   C: lane l holds C[4*(l/16) + i][l % 16]: its own sub-group (slot = kb),
//     th = i.  Seeded with (0, -8 sum xq) per token, the row pair gives
//     V = 256 C[hi] + C[lo] = sum_k (n_k - 8) xq_k exactly in int32, and the
//     lane adds s * sigma * V to the token's fp32 sum.
// The digits carry x to within sigma / 2 (2^-16 of the sub-group's largest
// magnitude); the products and their sums are exact integers, so the only
// roundings are that quantisation and the fp32 accumulation.
//
// LDS (see lpk::frag_lds_bytes): zero block, then per token pair p
//   frag[p][th][g] : 32 B (MFMA h = 0 bytes, then h = 1), g < ngp
//   off [p][g]     : int4 (0, seed of token 2p, 0, seed of token 2p + 1)
//   sig [p][g]     : float2 (sigma of token 2p, sigma of token 2p + 1)
// ---------------------------------------------------------------------------

typedef int i32x4_t __attribute__((ext_vector_type(4)));

struct Frags {
    uint8_t* lds;  // start of the fragment area (zero block first)
    int ng;        // sub-groups with data (cols / 32)
    int ngp;       // padded sub-groups (multiple of 4)
};

__device__ __forceinline__ Frags frags_at(uint8_t* lds, int cols) {
    Frags F;
    F.lds = lds;
    F.ng = cols >> 5;
    F.ngp = lpk::frag_ngp(cols);
    return F;
}

__device__ __forceinline__ uint8_t* pair_base(const Frags& F, int p) {
    return F.lds + lpk::kZeroBytes + p * lpk::frag_pair_bytes(F.ngp);
}

__device__ __forceinline__ uint8_t* frag_ptr(const Frags& F, int p, int th, int g) {
    return pair_base(F, p) + th * lpk::frag_th_stride(F.ngp) + g * 32;
}

__device__ __forceinline__ int32_t* off_ptr(const Frags& F, int p, int g) {
    return reinterpret_cast<int32_t*>(pair_base(F, p) + lpk::frag_off_bytes(F.ngp) + g * 16);
}

__device__ __forceinline__ float* sig_ptr(const Frags& F, int p, int g) {
    return reinterpret_cast<float*>(pair_base(F, p) + lpk::frag_sig_bytes(F.ngp) + g * 8);
}

// Zero the idle-lane block (once per workgroup, before the first barrier).
__device__ __forceinline__ void zero_block(const Frags& F, int tid, int nthreads) {
    for (int i = tid; i < lpk::kZeroBytes / 16; i += nthreads)
        reinterpret_cast<uint4*>(F.lds)[i] = make_uint4(0, 0, 0, 0);
}

// Column (within a 32-column sub-group) of digit byte t of MFMA h.
__device__ __forceinline__ constexpr int digit_col(int h, int t) {
    return 16 * h + 8 * (t >> 3) + 2 * (t & 3) + ((t >> 2) & 1);
}

// The largest magnitude below which a sub-group's digits are all zero (its
// contribution is below fp32's reach next to any other sub-group's).
constexpr float kDigitMin = 1.0e-30f;

// 16-bit fixed point of one value against inv = 32639 / m, as hi and lo
// digits; returns xq.
__device__ __forceinline__ int digit_split(float x, float inv, int& hi, int& lo) {
    const int xq = (int)rintf(x * inv);
    hi = (xq + 128) >> 8;
    lo = xq - (hi << 8);
    return xq;
}

__device__ __forceinline__ uint32_t pack_i8x4(int a, int b, int c, int d) {
    return (uint32_t)(a & 255) | ((uint32_t)(b & 255) << 8) | ((uint32_t)(c & 255) << 16) | ((uint32_t)d << 24);
}

// One 32-column sub-group of an fp32 row as digits in operand order, its
// seed -8 * sum xq and sigma.  p == 0 gives zeros (padding sub-groups,
// missing tokens).
struct DigitGroup {
    uint4 hi[2], lo[2];
    int32_t seed;
    float sigma;
};

__device__ __forceinline__ DigitGroup digit_group(const LP_GLOBAL float4* p) {
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float4 f = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (p) f = p[i];
        v[4 * i] = f.x;
        v[4 * i + 1] = f.y;
        v[4 * i + 2] = f.z;
        v[4 * i + 3] = f.w;
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(v[i]));
    DigitGroup q;
    const bool live = m >= kDigitMin;
    const float inv = live ? 32639.0f / m : 0.0f;
    q.sigma = live ? m / 32639.0f : 0.0f;
    int hi[32], lo[32], sum = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) sum += digit_split(v[i], inv, hi[i], lo[i]);
    q.seed = -8 * sum;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        uint32_t wh[4], wl[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int c0 = digit_col(h, 4 * w), c1 = digit_col(h, 4 * w + 1), c2 = digit_col(h, 4 * w + 2),
                      c3 = digit_col(h, 4 * w + 3);
            wh[w] = pack_i8x4(hi[c0], hi[c1], hi[c2], hi[c3]);
            wl[w] = pack_i8x4(lo[c0], lo[c1], lo[c2], lo[c3]);
        }
        q.hi[h] = make_uint4(wh[0], wh[1], wh[2], wh[3]);
        q.lo[h] = make_uint4(wl[0], wl[1], wl[2], wl[3]);
    }
    return q;
}

// Stage ntok activation rows into fragment pairs 0 .. ceil(ntok/2)-1.
// row_of(t) returns the f32 row of token t.  Work units (token, sub-group)
// are spread over the `nthreads` participating threads; a missing second
// token of the last pair and the padding sub-groups are written as zeros.
template <typename RowOf>
__device__ inline void stage_rows(const Frags& F, int ntok, RowOf row_of, int tid, int nthreads) {
    const int units = ((ntok + 1) & ~1) * F.ngp;
    for (int u = tid; u < units; u += nthreads) {
        const int t = u / F.ngp;
        const int g = u - t * F.ngp;
        const int pair = t >> 1, tk = t & 1;
        const bool live = t < ntok && g < F.ng;
        const DigitGroup q =
            digit_group(live ? gptr<float4>(reinterpret_cast<uint64_t>(row_of(t) + (size_t)g * 32)) : nullptr);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            *reinterpret_cast<uint4*>(frag_ptr(F, pair, 2 * tk + 0, g) + h * 16) = q.hi[h];
            *reinterpret_cast<uint4*>(frag_ptr(F, pair, 2 * tk + 1, g) + h * 16) = q.lo[h];
        }
        int32_t* of = off_ptr(F, pair, g);
        of[2 * tk + 0] = 0;
        of[2 * tk + 1] = q.seed;
        sig_ptr(F, pair, g)[tk] = q.sigma;
    }
}

// Sub-group g of an fp32 row of `cols` columns into the row's digit image
// (lpk::dimage_bytes layout).
__device__ __forceinline__ void write_dimage_group(const float* row, int cols, int g, uint8_t* img) {
    const int ng = cols >> 5, ngp = lpk::frag_ngp(cols);
    const DigitGroup q =
        digit_group(g < ng ? gptr<float4>(reinterpret_cast<uint64_t>(row + (size_t)g * 32)) : nullptr);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        reinterpret_cast<uint4*>(img + (size_t)g * 32)[h] = q.hi[h];
        reinterpret_cast<uint4*>(img + (size_t)ngp * 32 + (size_t)g * 32)[h] = q.lo[h];
    }
    reinterpret_cast<int2*>(img + lpk::dimage_seed_off(ngp))[g] = make_int2(0, q.seed);
    reinterpret_cast<float*>(img + lpk::dimage_sigma_off(ngp))[g] = q.sigma;
}

// fp16 images (lpk::himage_bytes layout), the token operand of the prefill
// GEMM.  The exponent e of a row (or act chunk) whose largest magnitude is m
// puts m 2^-e in [2^14, 2^15), so every value down to 2^-28 m stays a normal
// fp16; a zero or non-finite m gives e = 0 (zeros stay zero, inf and NaN
// carry through).
__device__ __forceinline__ int h16_exp(float m) {
    return m > 0.0f && m <= 3.402823466e38f ? __builtin_amdgcn_frexp_expf(m) - 15 : 0;
}

// Columns 8 j .. 8 j + 7 of a sub-group (v[0..7]) times 2^-e, rounded to fp16
// (RNE), as the image's 16-byte word j: halves in the order (0, 4, 1, 5, 2, 6,
// 3, 7), the order in which a q4 weight word unpacks.
__device__ __forceinline__ uint4 h16_word(const float (&v)[8], int e) {
    uint32_t h[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)__builtin_ldexpf(v[i], -e));
    return make_uint4(h[0] | (h[4] << 16), h[1] | (h[5] << 16), h[2] | (h[6] << 16), h[3] | (h[7] << 16));
}

// Largest |x| over columns 4 first, 4 (first + step), ... (four each) of an
// fp32 row (cols % 4 == 0, 16-byte aligned), reduced over the wave: the
// result in every lane.
__device__ __forceinline__ float row_absmax_wave(const float* row, int cols, int first, int step) {
    float m = 0.0f;
    for (int c = 4 * first; c < cols; c += 4 * step) {
        const float4 v = *reinterpret_cast<const float4*>(row + c);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    return m;
}

// Words first, first + step, ... of the fp16 image of an fp32 row with
// exponent e (zero words for the padding sub-groups).
__device__ __forceinline__ void write_h16_words(const float* row, int cols, int e, uint8_t* img, int first,
                                                int step) {
    const int ng = cols >> 5, nw = 4 * lpk::frag_ngp(cols);
    for (int w = first; w < nw; w += step) {
        const int g = w >> 2, j = w & 3;
        float v[8];
        if (g < ng) {
            const float4 f0 = *reinterpret_cast<const float4*>(row + g * 32 + j * 8);
            const float4 f1 = *reinterpret_cast<const float4*>(row + g * 32 + j * 8 + 4);
            v[0] = f0.x; v[1] = f0.y; v[2] = f0.z; v[3] = f0.w;
            v[4] = f1.x; v[5] = f1.y; v[6] = f1.z; v[7] = f1.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = 0.0f;
        }
        reinterpret_cast<uint4*>(img)[w] = h16_word(v, e);
    }
}

// The fp16 image of an fp32 row (global memory or LDS) and its exponent
// (*exp_out), by the whole workgroup (every thread calls it).
__device__ __forceinline__ void write_h16_image(const float* row, int cols, uint8_t* img, int* exp_out) {
    __shared__ float red[16];
    const int wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    float m = row_absmax_wave(row, cols, threadIdx.x, blockDim.x);
    if (lane_id() == 0) red[wave] = m;
    __syncthreads();
    for (int w = 0; w < nwaves; ++w) m = fmaxf(m, red[w]);
    __syncthreads();  // red is free for the next row
    const int e = h16_exp(m);
    write_h16_words(row, cols, e, img, threadIdx.x, blockDim.x);
    if (threadIdx.x == 0) *exp_out = e;
}

// Direct-to-LDS copy from inline assembly: lane l's 16 bytes at base + off
// land at LDS address lds + 16 l (base and lds uniform over the wave: an SGPR
// pair and M0).  Given the intrinsic instead, the compiler waits for every
// outstanding load before the first copy, which here would serialise the
// image copies behind a tile's weight loads; the callers wait explicitly.
__device__ __forceinline__ void lds_copy16(uint64_t base, uint32_t off, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}

// As lds_copy16 for 4 bytes per lane from per-lane 64-bit addresses.
__device__ __forceinline__ void lds_copy4(uint64_t addr, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(addr), "{m0}"(lds) : "memory");
}

__device__ __forceinline__ uint64_t uniform_u64(uint64_t v) {
    return (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v) |
           ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32)) << 32);
}

__device__ __forceinline__ uint32_t lds_addr_of(const uint8_t* p) {
    return (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)(uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p);
}

// Copy the digit images of nt tokens (img_of(t): device address of token t's
// image) into fragment pairs 0 .. ceil(nt/2)-1.  Digit blocks go straight
// from memory into LDS (64 lanes fill 1 KB per instruction, no registers, no
// LDS store), one instruction per wave in turn; the seeds and scales go
// through registers.  Ends with every load of the calling thread complete;
// the caller's barrier then publishes the copy.  The second token of an odd
// last pair is left as it is: its MFMA output rows are separate and never
// stored.
template <typename ImgOf>
__device__ inline void load_images(const Frags& F, int nt, ImgOf img_of) {
    const int lane = lane_id(), wave = threadIdx.x >> 6, W = blockDim.x >> 6;
    const int q4 = 2 * F.ngp;          // 16-byte units per digit block
    const int ipb = (q4 + 63) >> 6;    // DMA instructions per digit block
    for (int i = wave; i < 2 * nt * ipb; i += W) {
        const int blk = i / ipb, r = i - blk * ipb;  // blk = 2 * token + digit
        const int t = blk >> 1, part = blk & 1;
        const int q = r * 64 + lane;
        const uint64_t base = uniform_u64(img_of(t) + (uint64_t)part * F.ngp * 32 + (uint64_t)r * 1024);
        const uint32_t dst = lds_addr_of(frag_ptr(F, t >> 1, 2 * (t & 1) + part, 0) + r * 1024);
        if (q < q4) lds_copy16(base, (uint32_t)lane * 16u, dst);
    }
    for (int f = threadIdx.x; f < nt * F.ngp; f += blockDim.x) {
        const int t = f / F.ngp, g = f - t * F.ngp;
        const uint64_t img = img_of(t);
        const int2 sd = gptr<int2>(img + lpk::dimage_seed_off(F.ngp))[g];
        const float sg = gptr<float>(img + lpk::dimage_sigma_off(F.ngp))[g];
        reinterpret_cast<int2*>(off_ptr(F, t >> 1, g))[t & 1] = sd;
        sig_ptr(F, t >> 1, g)[t & 1] = sg;
    }
    __builtin_amdgcn_s_waitcnt(0);  // the LDS-direct loads have landed
}

// load_images without registers and without the final wait: the seeds and
// scales, too, are gathered straight into LDS (one 4-byte copy per lane:
// dword d of pair p's seed block is word (d & 1) of token 2p + ((d >> 1) & 1)
// at sub-group d >> 2, dword d of its scale block the scale of token
// 2p + (d & 1) at sub-group d >> 1; a missing second token repeats the
// first).  The caller waits for every load of the thread (vmcnt 0) before its
// barrier, so these may be issued ahead of other loads that the same wait
// then covers.
template <typename ImgOf>
__device__ inline void issue_images(const Frags& F, int nt, ImgOf img_of) {
    const int lane = lane_id(), wave = threadIdx.x >> 6, W = blockDim.x >> 6;
    const int q4 = 2 * F.ngp;          // 16-byte units per digit block
    const int ipb = (q4 + 63) >> 6;    // copies per digit block
    for (int i = wave; i < 2 * nt * ipb; i += W) {
        const int blk = i / ipb, r = i - blk * ipb;  // blk = 2 * token + digit
        const int t = blk >> 1, part = blk & 1;
        const uint64_t base = uniform_u64(img_of(t) + (uint64_t)part * F.ngp * 32 + (uint64_t)r * 1024);
        const uint32_t dst = lds_addr_of(frag_ptr(F, t >> 1, 2 * (t & 1) + part, 0) + r * 1024);
        if (r * 64 + lane < q4) lds_copy16(base, (uint32_t)lane * 16u, dst);
    }
    const int npair = (nt + 1) >> 1;
    const int spp = (F.ngp * 4 + 63) >> 6;  // seed copies per pair
    for (int i = wave; i < npair * spp; i += W) {
        const int p = i / spp, r = i - p * spp;
        const int d = r * 64 + lane;
        const int g = d >> 2;
        const int t = min(2 * p + ((d >> 1) & 1), nt - 1);
        const uint32_t dst = lds_addr_of(reinterpret_cast<const uint8_t*>(off_ptr(F, p, 0)) + r * 256);
        if (g < F.ngp)
            lds_copy4(img_of(t) + (uint64_t)lpk::dimage_seed_off(F.ngp) + (uint64_t)g * 8 + (uint64_t)(d & 1) * 4,
                      dst);
    }
    const int gpp = (F.ngp * 2 + 63) >> 6;  // scale copies per pair
    for (int i = wave; i < npair * gpp; i += W) {
        const int p = i / gpp, r = i - p * gpp;
        const int d = r * 64 + lane;
        const int g = d >> 1;
        const int t = min(2 * p + (d & 1), nt - 1);
        const uint32_t dst = lds_addr_of(reinterpret_cast<const uint8_t*>(sig_ptr(F, p, 0)) + r * 256);
        if (g < F.ngp) lds_copy4(img_of(t) + (uint64_t)lpk::dimage_sigma_off(F.ngp) + (uint64_t)g * 4, dst);
    }
}

__device__ __forceinline__ int tile_steps(int cols) { return ((cols >> 5) + 3) >> 2; }

// One 16-row tile of a q4 region [rows, cols] (scales then nibbles, the blob
// layout), read through a raw buffer resource that covers exactly the
// region: loads past its end return zeros instead of faulting, so no lane
// ever needs a clamped address.  Lane (n, kb) owns row n0 + n and, at step c,
// sub-group 4c + kb (64 contiguous bytes per row and step over the four kb
// lanes).  One f16 scale covers 2^RS sub-groups (group = 32 << RS, RS <= 2).
template <int RS>
struct WTile {
    __amdgpu_buffer_rsrc_t rsrc;
    uint64_t base;  // the region's address (the rsrc's base)
    uint32_t dofs;  // lane's nibble byte offset at step 0
    uint32_t sofs;  // lane's scale byte offset at step 0
    bool lastok;    // the lane's sub-group exists at the tile's last step
};

template <int RS>
__device__ __forceinline__ WTile<RS> wtile(uint64_t region, int rows, int cols, int n0) {
    const int lane = lane_id();
    const int n = lane & 15, kb = lane >> 4;
    const uint32_t ng = (uint32_t)cols >> 5, gpr = ng >> RS;
    const uint32_t sbytes = (uint32_t)rows * gpr * 2;
    const uint32_t row = (uint32_t)(n0 + n);
    WTile<RS> T;
    T.rsrc = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(region), (short)0,
                                               (int)(sbytes + (uint32_t)rows * ng * 16), kBufferWord3);
    T.base = region;
    T.dofs = sbytes + (row * ng + kb) * 16;
    T.sofs = (row * gpr + (kb >> RS)) * 2;
    T.lastok = (ng & 3) == 0 || kb < (int)(ng & 3);
    return T;
}

// Raw weight registers for steps [c0, c0 + NS) of one tile.  Rows past the
// matrix read zero nibbles (past the buffer) and garbage scales; their
// outputs are never stored, so they need no mask.
//
// Scales: per lane one 16-bit load per step (SL false), or (SL true: group
// 32, one chunk from step 0, rows' scales 16-byte aligned) the tile's scale
// lines copied straight into a per-wave LDS window, 2 NS bytes per lane:
// lane (n, kb') copies bytes [2 NS kb', 2 NS (kb' + 1)) of row n's scales,
// 16 at a time, the i-th 16 landing at window + 1024 i + 16 lane.  Scale q
// (= 4 c + kb at step c) of row n then sits at window + 1024 ((q % NS) / 8) +
// 16 (n + 16 (q / NS)) + 2 (q % 8): a per-lane base plus a constant per step.
// Here NS is the window's width, window_steps<NS>(): the chunk's steps
// rounded up to a multiple of 8, so that a chunk of 6 or 12 steps loads only
// its own nibbles and still copies whole 16-byte scale lines.
// The per-lane loads touch 16 cache lines per instruction for 128 useful
// bytes; the window copy reads each line once.
template <int NS>
__host__ __device__ constexpr int window_steps() { return (NS + 7) / 8 * 8; }

template <int NS, bool SL = false>
struct WRegs {
    uint4 w[NS];
    // f16 bits of the lane's sub-group scale (SL false), kept 16-bit: a
    // widening right after the load would make the wave wait for it there
    uint16_t s[SL ? 1 : NS];
    uint32_t sbase;  // SL: LDS address of the lane's scale at step 0
    bool lastok;     // the lane's sub-group exists at the tile's last step
};

// LDS byte offset of step j's scale from WRegs::sbase (SL) in a window NW
// steps wide.
template <int NW>
__device__ __forceinline__ constexpr uint32_t scale_step_off(int j) {
    return 1024u * (uint32_t)(((4 * j) % NW) / 8) + 256u * (uint32_t)((4 * j) / NW) + 8u * (uint32_t)(j & 1);
}

// Issue the tile's loads for steps c0 .. c0 + NS - 1: one per-lane offset
// plus an immediate per step (64 B of nibbles, 8 >> RS B of scales).  The
// loads are unconditional, so the compiler keeps them together ahead of
// their use.  Steps past the lane's last sub-group read whatever follows in
// the region (or zeros past its end); wmma gives them a zero scale.  SL:
// c0 is 0 and swin is the wave's LDS window for this tile (64 * 2 NS bytes);
// the copies are waited for by the caller's wait for all loads.
template <int NS, int RS, bool SL>
__device__ __forceinline__ void wload(WRegs<NS, SL>& R, const WTile<RS>& T, int c0, uint32_t swin = 0) {
    R.lastok = T.lastok;
    uint32_t d = T.dofs + 64u * (uint32_t)c0;
    uint32_t sc = T.sofs + (8u >> RS) * (uint32_t)c0;
    // opaque per-chunk bases: every step is then base + immediate, and the
    // compiler cannot hoist NS separate step addresses out of a chunk loop
    asm volatile("" : "+v"(d), "+v"(sc));
    if constexpr (SL) {
        static_assert(RS == 0, "LDS scales: group 32");
        constexpr int NW = window_steps<NS>();
        const int lane = lane_id(), kb = lane >> 4;
        const uint32_t row0 = T.sofs - 2u * (uint32_t)kb;  // the row's first scale
        const uint64_t base = uniform_u64(T.base);
#pragma unroll
        for (int i = 0; i < NW / 8; ++i)
            lds_copy16(base, row0 + 2u * NW * (uint32_t)kb + 16u * (uint32_t)i, swin + 1024u * (uint32_t)i);
        R.sbase = swin + 16u * (uint32_t)(lane & 15) + 2u * (uint32_t)kb;
    }
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        R.w[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(T.rsrc, (int)(d + 64u * j), 0, 0));
        if constexpr (!SL) R.s[j] = __builtin_amdgcn_raw_buffer_load_b16(T.rsrc, (int)(sc + (8u >> RS) * j), 0, 0);
    }
}

// Make a chunk's registers opaque to the optimiser.  Called where a chunk
// is reused (each token group of a tile that stays in registers): without
// it the decoded bf16 weights, invariant across the groups, are hoisted out
// of the group loop and take four registers per loaded one.  Emits no code;
// the loads must already be complete (they are, after load_images).
template <int NS, bool SL>
__device__ __forceinline__ void opaque(WRegs<NS, SL>& R) {
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        asm volatile("" : "+v"(R.w[j].x), "+v"(R.w[j].y), "+v"(R.w[j].z), "+v"(R.w[j].w));
        if constexpr (!SL) asm volatile("" : "+v"(R.s[j]));
    }
}

// Per-lane LDS bases for the A operand, the accumulator seeds and the token
// scales of pair p at step chunk c0 (steps are 128 B apart in frag, 64 B in
// off, 32 B in sig).
struct ABase {
    const uint8_t* a;
    const uint8_t* o;
    const uint8_t* sg;
};

__device__ __forceinline__ ABase abase(const Frags& F, int p, int c0) {
    const int lane = lane_id();
    const int kb = lane >> 4, m = lane & 15;
    const bool live = (m >> 2) == kb;  // A lane (m, kb) is live when its slot m/4 == kb
    ABase b;
    b.a = live ? frag_ptr(F, p, m & 3, 4 * c0 + kb) : F.lds;
    b.o = reinterpret_cast<const uint8_t*>(off_ptr(F, p, 4 * c0 + kb));
    b.sg = reinterpret_cast<const uint8_t*>(sig_ptr(F, p, 4 * c0 + kb));
    return b;
}

// The two B operands of one 16-byte nibble load: bytes in digit_col order.
__device__ __forceinline__ void q4_digits(const uint4& w, i32x4_t& b0, i32x4_t& b1) {
    b0 = i32x4_t{(int)(w.x & 0x0F0F0F0Fu), (int)((w.x >> 4) & 0x0F0F0F0Fu), (int)(w.y & 0x0F0F0F0Fu),
                 (int)((w.y >> 4) & 0x0F0F0F0Fu)};
    b1 = i32x4_t{(int)(w.z & 0x0F0F0F0Fu), (int)((w.z >> 4) & 0x0F0F0F0Fu), (int)(w.w & 0x0F0F0F0Fu),
                 (int)((w.w >> 4) & 0x0F0F0F0Fu)};
}

// MFMAs of one loaded chunk for M weight tiles that share the same staged
// activations (gate and up of one expert, or several row tiles of one
// matrix) against the first np (<= P) token pairs: acc[m][p][0..1] +=
// tokens 2p, 2p+1 of tile m.  Every step reads the A fragments once for all
// M tiles, and the M independent MFMA chains interleave.  rem = steps left
// in the tile from this chunk: steps j >= rem are skipped (uniform branch),
// and at step rem - 1 lanes without a sub-group (cols % 128 != 0) take a
// zero scale.  One code path serves every np, so the loaded chunk keeps its
// registers whatever the token count.  NF > 0 instead takes exactly the
// first NF pairs (np unused): no branch between pairs, so their MFMA chains
// interleave.
template <int NS, bool SL, int P, int M, int NF = 0>
__device__ __forceinline__ void wmma(const WRegs<NS, SL> (&R)[M], const ABase (&B)[P], int rem, int np,
                                     float (&acc)[M][P][2]) {
    static_assert(NF <= P, "NF pairs of at most P");
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        if (j < rem) {  // uniform
            float s[M];
            i32x4_t b[M][2];
#pragma unroll
            for (int m = 0; m < M; ++m) {
                if constexpr (SL)
                    s[m] = f16_bits_to_f32(*reinterpret_cast<const __attribute__((address_space(3))) uint16_t*>(
                        (uintptr_t)(R[m].sbase + scale_step_off<window_steps<NS>()>(j))));
                else
                    s[m] = f16_bits_to_f32(R[m].s[j]);
                if (j == rem - 1 && !R[m].lastok) s[m] = 0.0f;
                q4_digits(R[m].w[j], b[m][0], b[m][1]);
            }
#pragma unroll
            for (int p = 0; p < (NF > 0 ? NF : P); ++p) {
                if (NF == 0 && p > 0 && p >= np) break;  // uniform: pairs staged in this token group
                const i32x4_t o = *reinterpret_cast<const i32x4_t*>(B[p].o + j * 64);
                const float2 sg = *reinterpret_cast<const float2*>(B[p].sg + j * 32);
                const i32x4_t a0 = *reinterpret_cast<const i32x4_t*>(B[p].a + j * 128);
                const i32x4_t a1 = *reinterpret_cast<const i32x4_t*>(B[p].a + j * 128 + 16);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    i32x4_t c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b[m][0], o, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b[m][1], c, 0, 0, 0);
                    const int v0 = (c[0] << 8) + c[1], v1 = (c[2] << 8) + c[3];
                    acc[m][p][0] = __builtin_fmaf(s[m] * sg.x, (float)v0, acc[m][p][0]);
                    acc[m][p][1] = __builtin_fmaf(s[m] * sg.y, (float)v1, acc[m][p][1]);
                }
            }
        }
        // keep each step's LDS reads next to their MFMAs: hoisting all of them
        // to the top of the chunk costs more registers than the latency saves
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Sum the four kb partials of row n: afterwards every lane (n, *) holds the row.
__device__ __forceinline__ float tile_reduce(float v) {
    v += shfl_xor(v, 16);
    v += shfl_xor(v, 32);
    return v;
}

// The same sums for several tokens at once, by register swaps between lanes
// (no LDS round trip), each token's sum landing in one row of 16 lanes.
// pair_rows(a, b): rows 0 and 1 hold a's partials of rows {0, 2} and {1, 3},
// rows 2 and 3 the same of b (v_permlane32_swap trades the first operand's
// upper 32 lanes for the second's lower 32).
__device__ __forceinline__ float pair_rows(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// quad_rows(pair_rows(a, b), pair_rows(c, d)): rows 0, 1, 2, 3 hold the full
// sums of a, c, b, d (v_permlane16_swap trades the first operand's odd rows
// for the second's even rows).
__device__ __forceinline__ float quad_rows(float s, float t) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(t), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Token (0..3, of a, b = tokens 0, 1 and c, d = tokens 2, 3) in row r of a
// quad_rows result.
__device__ __forceinline__ constexpr int quad_row_tok(int r) { return 2 * (r & 1) + (r >> 1); }

__device__ __forceinline__ int ilog2_pow2(int v) { return 31 - __builtin_clz(v); }

}  // namespace lp
