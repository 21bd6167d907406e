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
// MFMA v_mfma_f32_16x16x32_bf16 (C[m][n] += sum_k A[m][k] B[k][n]):
//   B (weights): lane l = (n = l % 16, kb = l / 16).  At step c the four
//     lanes of row n load sub-groups 4c..4c+3 (64 contiguous bytes of the row,
//     16 per lane); MFMA d (0..3) takes the d-th 32-bit word of each load.
//   A (activations): row m = 4*slot + th, th = 2*token + part, part 0 =
//     bf16(x), part 1 = bf16(x - bf16(x)).  Element (m, k = 8*kbA + i) is
//     non-zero only when slot == kbA, so the 16 MFMA output rows keep four
//     sub-groups x four (token, part) apart.  Lanes whose slot is not their
//     kb read a zero block, so every LDS read is unconditional.
//   C: lane l holds C[4*(l/16) + i][l % 16]: its own sub-group (slot = kb),
//     th = i.  With n = q + 8 the stored nibble, the weight operand is
//     128 + n, so sum_k (128 + n_k) x_k = sum_k (n_k - 8) x_k + 136 sum_k x_k;
//     the accumulator is therefore seeded with -136 * sum_k x_k of the part.
// Products of bf16 values are exact in fp32 and x = part0 + part1 to 16
// significant bits, so the only roundings are the fp32 accumulations.
//
// LDS (see lpk::frag_lds_bytes): zero block, then per token pair p
//   frag[p][th][g][d] : uint4 (8 bf16 in element order i), g < ngp
//   off [p][g][th]    : float, -136 * sum of the th part over sub-group g
// ---------------------------------------------------------------------------

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

__device__ __forceinline__ uint8_t* frag_ptr(const Frags& F, int p, int th, int g) {
    return F.lds + lpk::kZeroBytes + p * lpk::frag_pair_bytes(F.ngp) + th * lpk::frag_th_stride(F.ngp) + g * 64;
}

__device__ __forceinline__ float* off_ptr(const Frags& F, int p, int g) {
    return reinterpret_cast<float*>(F.lds + lpk::kZeroBytes + p * lpk::frag_pair_bytes(F.ngp) +
                                    4 * lpk::frag_th_stride(F.ngp) + g * 16);
}

// Zero the idle-lane block (once per workgroup, before the first barrier).
__device__ __forceinline__ void zero_block(const Frags& F, int tid, int nthreads) {
    for (int i = tid; i < lpk::kZeroBytes / 16; i += nthreads)
        reinterpret_cast<uint4*>(F.lds)[i] = make_uint4(0, 0, 0, 0);
}

// One 32-column sub-group of an fp32 row as fragment words: the bf16 parts
// hi = bf16(x) and lo = bf16(x - hi) in fragment order (32-bit word w of
// uint4 d pairs columns 8d + w and 8d + w + 4) and each part's sum.  p == 0
// gives zeros (padding sub-groups, missing tokens).
struct GroupFrag {
    uint4 hi[4], lo[4];
    float shi, slo;
};

__device__ __forceinline__ GroupFrag convert_group(const LP_GLOBAL float4* p) {
    GroupFrag q;
    q.shi = 0.0f;
    q.slo = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        float v[8];
        if (p) {
            const float4 f0 = p[2 * d], f1 = p[2 * d + 1];
            v[0] = f0.x; v[1] = f0.y; v[2] = f0.z; v[3] = f0.w;
            v[4] = f1.x; v[5] = f1.y; v[6] = f1.z; v[7] = f1.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = 0.0f;
        }
        uint32_t hi[8], lo[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            hi[i] = f32_to_bf16_rne(v[i]);
            lo[i] = f32_to_bf16_rne(v[i] - bf16_to_f32(hi[i]));
            q.shi += bf16_to_f32(hi[i]);
            q.slo += bf16_to_f32(lo[i]);
        }
        q.hi[d] = make_uint4(hi[0] | (hi[4] << 16), hi[1] | (hi[5] << 16), hi[2] | (hi[6] << 16),
                             hi[3] | (hi[7] << 16));
        q.lo[d] = make_uint4(lo[0] | (lo[4] << 16), lo[1] | (lo[5] << 16), lo[2] | (lo[6] << 16),
                             lo[3] | (lo[7] << 16));
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
        const GroupFrag q =
            convert_group(live ? gptr<float4>(reinterpret_cast<uint64_t>(row_of(t) + (size_t)g * 32)) : nullptr);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            *reinterpret_cast<uint4*>(frag_ptr(F, pair, 2 * tk + 0, g) + d * 16) = q.hi[d];
            *reinterpret_cast<uint4*>(frag_ptr(F, pair, 2 * tk + 1, g) + d * 16) = q.lo[d];
        }
        float* of = off_ptr(F, pair, g);
        of[2 * tk + 0] = -136.0f * q.shi;
        of[2 * tk + 1] = -136.0f * q.slo;
    }
}

// Sub-group g of an fp32 row of `cols` columns into the row's fragment image
// (lpk::image_bytes layout): part blocks [2][ngp][64 B], then seeds [ngp][2]:
// [0] = -136 * sum(hi) + -136 * sum(lo), the whole sub-group's seed, and
// [1] = 0 (a consumer that keeps the parts in separate accumulator rows seeds
// the hi row with [0] and the lo row with [1]).  Returns whether any lo
// element is non-zero.
__device__ __forceinline__ bool write_image_group(const float* row, int cols, int g, uint8_t* img) {
    const int ng = cols >> 5, ngp = lpk::frag_ngp(cols);
    const GroupFrag q =
        convert_group(g < ng ? gptr<float4>(reinterpret_cast<uint64_t>(row + (size_t)g * 32)) : nullptr);
    uint4* hi = reinterpret_cast<uint4*>(img + (size_t)g * 64);
    uint4* lo = reinterpret_cast<uint4*>(img + (size_t)ngp * 64 + (size_t)g * 64);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        hi[d] = q.hi[d];
        lo[d] = q.lo[d];
    }
    reinterpret_cast<float2*>(img + (size_t)ngp * 128)[g] = make_float2(-136.0f * q.shi + -136.0f * q.slo, 0.0f);
    uint32_t any = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) any |= q.lo[d].x | q.lo[d].y | q.lo[d].z | q.lo[d].w;
    return any != 0;
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

// Copy the fragment images of nt tokens (img_of(t): device address of token
// t's image) into fragment pairs 0 .. ceil(nt/2)-1.  Part blocks go straight
// from memory into LDS (64 lanes fill 1 KB per instruction, no registers, no
// LDS store), one instruction per wave in turn; the seeds go through
// registers.  Ends with every load of the calling thread complete; the
// caller's barrier then publishes the copy.  The second token of an odd last
// pair is left as it is: its MFMA output rows are separate and never stored.
template <typename ImgOf>
__device__ inline void load_images(const Frags& F, int nt, ImgOf img_of) {
    const int lane = lane_id(), wave = threadIdx.x >> 6, W = blockDim.x >> 6;
    const int q4 = 4 * F.ngp;          // 16-byte units per part block
    const int ipb = (q4 + 63) >> 6;    // DMA instructions per part block
    for (int i = wave; i < 2 * nt * ipb; i += W) {
        const int blk = i / ipb, r = i - blk * ipb;  // blk = 2 * token + part
        const int t = blk >> 1, part = blk & 1;
        const int q = r * 64 + lane;
        const uint64_t base = uniform_u64(img_of(t) + (uint64_t)part * F.ngp * 64 + (uint64_t)r * 1024);
        const uint32_t dst = lds_addr_of(frag_ptr(F, t >> 1, 2 * (t & 1) + part, 0) + r * 1024);
        if (q < q4) lds_copy16(base, (uint32_t)lane * 16u, dst);
    }
    for (int f = threadIdx.x; f < nt * F.ngp; f += blockDim.x) {
        const int t = f / F.ngp, g = f - t * F.ngp;
        const uint2 sd = gptr<uint2>(img_of(t) + (uint64_t)F.ngp * 128)[g];
        *reinterpret_cast<uint2*>(reinterpret_cast<uint8_t*>(off_ptr(F, t >> 1, g)) + (t & 1) * 8) = sd;
    }
    __builtin_amdgcn_s_waitcnt(0);  // the LDS-direct loads have landed
}

// load_images without registers and without the final wait: the seeds, too,
// are gathered straight into LDS (one 4-byte copy per lane: dword d of pair
// p's seed block is seed (d & 1) of token 2p + ((d >> 1) & 1) at sub-group
// d >> 2; a missing second token repeats the first).  The caller waits for
// every load of the thread (vmcnt 0) before its barrier, so these may be
// issued ahead of other loads that the same wait then covers.
template <typename ImgOf>
__device__ inline void issue_images(const Frags& F, int nt, ImgOf img_of) {
    const int lane = lane_id(), wave = threadIdx.x >> 6, W = blockDim.x >> 6;
    const int q4 = 4 * F.ngp;          // 16-byte units per part block
    const int ipb = (q4 + 63) >> 6;    // copies per part block
    for (int i = wave; i < 2 * nt * ipb; i += W) {
        const int blk = i / ipb, r = i - blk * ipb;  // blk = 2 * token + part
        const int t = blk >> 1, part = blk & 1;
        const uint64_t base = uniform_u64(img_of(t) + (uint64_t)part * F.ngp * 64 + (uint64_t)r * 1024);
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
        if (g < F.ngp) lds_copy4(img_of(t) + (uint64_t)F.ngp * 128 + (uint64_t)g * 8 + (uint64_t)(d & 1) * 4, dst);
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

// Per-lane LDS bases for the A operand and the accumulator seeds of pair p
// at step chunk c0 (steps are 256 B apart in frag, 64 B apart in off).
struct ABase {
    const uint8_t* a;
    const uint8_t* o;
};

__device__ __forceinline__ ABase abase(const Frags& F, int p, int c0) {
    const int lane = lane_id();
    const int kb = lane >> 4, m = lane & 15;
    const bool live = (m >> 2) == kb;  // A lane (m, kb) is live when its slot m/4 == kb
    ABase b;
    b.a = live ? frag_ptr(F, p, m & 3, 4 * c0 + kb) : F.lds;
    b.o = reinterpret_cast<const uint8_t*>(off_ptr(F, p, 4 * c0 + kb));
    return b;
}

// MFMAs of one loaded chunk for M weight tiles that share the same staged
// activations (gate and up of one expert, or several row tiles of one
// matrix) against the first np (<= P) token pairs: acc[m][p][0..1] +=
// tokens 2p, 2p+1 of tile m.  Every step reads the A fragments once for all
// M tiles, and the M independent MFMA chains interleave.  rem = steps left
// in the tile from this chunk: steps j >= rem are skipped (uniform branch),
// and at step rem - 1 lanes without a sub-group (cols % 128 != 0) take a
// zero scale.  One code path serves every np, so the loaded chunk keeps its
// registers whatever the token count.
template <int NS, bool SL, int P, int M>
__device__ __forceinline__ void wmma(const WRegs<NS, SL> (&R)[M], const ABase (&B)[P], int rem, int np,
                                     float (&acc)[M][P][2]) {
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        if (j < rem) {  // uniform
            float s[M];
#pragma unroll
            for (int m = 0; m < M; ++m) {
                if constexpr (SL)
                    s[m] = f16_bits_to_f32(*reinterpret_cast<const __attribute__((address_space(3))) uint16_t*>(
                        (uintptr_t)(R[m].sbase + scale_step_off<window_steps<NS>()>(j))));
                else
                    s[m] = f16_bits_to_f32(R[m].s[j]);
                if (j == rem - 1 && !R[m].lastok) s[m] = 0.0f;
            }
#pragma unroll
            for (int p = 0; p < P; ++p) {
                if (p > 0 && p >= np) break;  // uniform: pairs staged in this token group
                const float4 o = *reinterpret_cast<const float4*>(B[p].o + j * 64);
                f32x4_t c[M];
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    c[m][0] = o.x;
                    c[m][1] = o.y;
                    c[m][2] = o.z;
                    c[m][3] = o.w;
                }
                // one A fragment and one decoded weight word per MFMA keeps
                // the step's temporaries to a few registers beside the chunk
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const uint4 a = *reinterpret_cast<const uint4*>(B[p].a + j * 256 + d * 16);
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const uint32_t w = d == 0 ? R[m].w[j].x : d == 1 ? R[m].w[j].y
                                         : d == 2 ? R[m].w[j].z : R[m].w[j].w;
                        c[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8_t, a), q4_word_to_bf16x8(w), c[m], 0, 0, 0);
                    }
                }
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    acc[m][p][0] = __builtin_fmaf(s[m], c[m][0] + c[m][1], acc[m][p][0]);
                    acc[m][p][1] = __builtin_fmaf(s[m], c[m][2] + c[m][3], acc[m][p][1]);
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

__device__ __forceinline__ int ilog2_pow2(int v) { return 31 - __builtin_clz(v); }

}  // namespace lp
