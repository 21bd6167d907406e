// Prefill: the grouped expert projections as MFMA GEMMs over the dispatch
// tables (the reference prefills with one GEMV per token, decode.rs:469-531;
// the arithmetic each output restates is q4g64.cu:19-81's).
//
// A tile is (routed expert, block of kGemmBM = 128 of its tokens, block of
// weight rows): gate/up tiles take 64 rows of gate and the same 64 rows of up
// so that SiLU * up is the epilogue; down tiles take 128 rows.  Wave w owns
// the 16-token blocks 2 mt + (w & 1), mt = 0..3, and one half of the rows
// (w >> 1): 4 x 4 tiles of v_mfma_f32_16x16x32_bf16 (gate/up: two gate tiles
// and the matching two up tiles).
//
// K runs over 32-column sub-groups, one pipeline stage each.  Operands reach
// LDS by direct-to-LDS loads (no registers, no LDS stores), each stream in
// whole 64-byte pieces of memory:
//   A: per stage, the 128 token rows' fragment blocks (bf16 hi = bf16(x), lo
//      = bf16(x - hi), in MFMA operand order; gate/up gathers the token images
//      through the dispatch permutation), lo only when a token of the tile has
//      one; three slots, loads two stages ahead;
//   B: per kGemmBGroups stages, 64 nibble bytes of each of the tile's 128
//      weight rows; two slots;
//   scales: per kGemmSGroups stages, a 16-scale window of each row; two slots.
// Each wave turns its B words into bf16 128 + q (one v_bitop3_b32 per two
// values); one MFMA of the A block against bf16(-136) gives -136 sum_k (hi +
// lo)_k, which seeds the sub-group's MFMAs, so they return sum_k x_k (q_k - 8)
// exactly up to fp32 rounding; the sub-group's scale is then applied in fp32.
#include "lp_device.h"

using namespace lp;
using namespace lpk;

namespace {

template <typename T>
__device__ __forceinline__ T* dptr(uint64_t a) {
    return reinterpret_cast<T*>(a);
}

__device__ __forceinline__ ExpertEntry load_entry(uint64_t et, int u) {
    const LP_GLOBAL uint4* p = gptr<uint4>(et + (uint64_t)u * sizeof(ExpertEntry));
    const uint4 lo = p[0], hi = p[1];
    ExpertEntry x;
    x.blob = (uint64_t)lo.x | ((uint64_t)lo.y << 32);
    x.p0 = (int)lo.z;
    x.ntok = (int)lo.w;
    x.tok[0] = (int)hi.x;
    x.tok[1] = (int)hi.y;
    x.tok[2] = (int)hi.z;
    x.tok[3] = (int)hi.w;
    return x;
}

__shared__ __align__(16) uint8_t g_lds[kGemmLds];

// Chunk kb (16 bytes) of token m's 64-byte block within a 16-token block of
// LDS sits at slot 4 m + (kb ^ chunk_swz(m)): the MFMA operand read (lane =
// 16 kb + m) then touches 16 distinct 16-byte bank groups per 16 lanes and 8
// per 8 lanes, while each direct-load quad still copies one token's 64
// contiguous bytes.
__device__ __forceinline__ int chunk_swz(int m) { return ((m >> 1) ^ (m >> 3)) & 3; }

// B slot: row r's kGemmBGroups 16-byte sub-group pieces sit at 64 r + 16 (j ^
// b_swz(r)) for sub-group j of the load, so that the operand read (16 rows x
// one 32-bit word) hits distinct banks; each direct-load quad still copies
// one row's 64 contiguous bytes.
__device__ __forceinline__ int b_swz(int r) { return (r >> 2) & 3; }

__device__ __forceinline__ void dma16(uint64_t base, uint32_t off, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}

// LDS address of g_lds (the M0 operand of the direct loads is an LDS address).
__device__ __forceinline__ uint32_t lds_base() {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)g_lds;
}

// Wait until at most n vector-memory loads of this wave are outstanding and
// its LDS reads are done; with the loads completing in issue order this is
// "stage s has landed" when n counts the loads issued after stage s's.
#define LP_WAIT_VM_LGKM0(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4))

// s_barrier as a compiler-level memory fence too: no LDS access or load moves
// across it.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_barrier" ::: "memory"); }

struct GemmTile {
    ExpertEntry x;
    int m0, mvalid, n0;   // token block start and size; first matrix row of the tile
    int K, NR, ng, ngp;   // reduction width, matrix rows, sub-groups, padded sub-groups
    uint64_t off0, off1;  // byte offsets in the blob: gate/up: gate and up regions; down: down twice
};

// Matrix row (in 0 .. NR-1) behind row r of the tile's B buffer.
template <int MODE>
__device__ __forceinline__ int tile_row(const GemmTile& g, int r) {
    return min(g.n0 + (MODE == 0 ? (r & 63) : r), g.NR - 1);
}

// Sum over the 16 lanes of a row, in every lane of the row: quad_perm
// [1,0,3,2] and [2,3,0,1], then row_half_mirror and row_mirror.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    return v + dpp_f<0x140>(v);
}

template <int MODE, int RS, bool LO>
__device__ __forceinline__ void gemm_main(const GemmArgs& a, const GemmTile& G) {
    // Sub-groups per stage: an A slot holds one sub-group's hi and lo parts,
    // or two sub-groups' hi parts when the tile has no lo.
    constexpr int GPS = LO ? 1 : 2;
    constexpr int OPS_A = 4;  // A loads per wave per stage (two 16-token blocks x two parts / sub-groups)
    const int tid = threadIdx.x, lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: DMA targets stay scalar
    const int wm = wave & 1, wn = wave >> 1;
    const int nst = (G.ng + GPS - 1) / GPS;
    const uint32_t lds0 = lds_base();
    const uint64_t part_bytes = (uint64_t)G.ngp * 64;
    const int gpr = G.ng >> RS;
    const uint32_t sbytes = (uint32_t)G.NR * gpr * 2;
    const uint64_t* rowimg = reinterpret_cast<const uint64_t*>(g_lds + kGemmLdsRows);

    // --- load sources: a uniform 64-bit base plus per-lane 32-bit offsets ---
    const uint64_t a_base = a.a_img;
    // (each half zero-extended: readfirstlane returns a signed int)
    const uint64_t w_base = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)G.x.blob) |
                            ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(G.x.blob >> 32)) << 32);
    // A: block 2 w + j of 16 tokens; lane l copies chunk (l & 3) ^ swz of token l >> 2
    uint32_t a_off[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int m = lane >> 2;
        a_off[j] = (uint32_t)(rowimg[16 * (2 * wave + j) + m] - a_base) + (uint32_t)(((lane & 3) ^ chunk_swz(m)) * 16);
    }
    // B: rows 32 w + 16 i + (l >> 2); lane l copies the row's piece j = l & 3,
    // i.e. sub-group kGemmBGroups S + (j ^ b_swz(row)) of load S
    uint32_t b_row[2];
    const int b_j = (lane & 3) ^ ((lane >> 4) & 3);  // j ^ b_swz(row): row bits 2-3 are lane bits 4-5
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = 32 * wave + 16 * i + (lane >> 2);
        const uint32_t mat = (uint32_t)((MODE == 0 && r >= 64) ? G.off1 : G.off0);
        b_row[i] = mat + sbytes + (uint32_t)tile_row<MODE>(G, r) * G.ng * 16;
    }
    // scales: row 32 w + (l >> 1), 16-byte half l & 1 of the row's window
    const int s_r = 32 * wave + (lane >> 1);
    const uint32_t s_mat = (uint32_t)((MODE == 0 && s_r >= 64) ? G.off1 : G.off0) + 16 * (lane & 1);
    const uint32_t s_idx = (uint32_t)tile_row<MODE>(G, s_r) * gpr;

    // stage st into A slot `slot`: half q of the slot is part q of sub-group
    // st (LO) or sub-group 2 st + q (no lo; a padding sub-group of the image
    // past the last one reads as zeros)
    auto issue_a = [&](int st, int slot) {
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                dma16(a_base + (LO ? q * part_bytes + (uint64_t)st * 64 : (uint64_t)(GPS * st + q) * 64), a_off[j],
                      lds0 + slot * kGemmSlotA + q * kGemmBM * 64 + (2 * wave + j) * 1024);
    };
    auto issue_b = [&](int S, int slot) {
        const uint32_t g = (uint32_t)min(kGemmBGroups * S + b_j, G.ng - 1);
#pragma unroll
        for (int i = 0; i < 2; ++i)
            dma16(w_base, b_row[i] + g * 16, lds0 + kGemmLdsB + slot * kGemmSlotB + (32 * wave + 16 * i) * 64);
    };
    // the window starts at the 8-aligned scale index at or below the row's
    // first scale of the load: 16 scales cover the 8 >> RS it needs
    auto issue_s = [&](int S, int slot) {
        const uint32_t c0 = (s_idx + (uint32_t)((kGemmSGroups * S) >> RS)) & ~7u;
        dma16(w_base, s_mat + c0 * 2, lds0 + kGemmLdsS + slot * kGemmSlotS + wave * 1024);
    };

    // --- read side ---
    // B / scale row of n-tile t: rbase + roff(t)
    const int rbase = MODE == 0 ? 32 * wn + (lane & 15) : 64 * wn + (lane & 15);
    auto roff = [](int t) { return MODE == 0 ? (t < 2 ? 16 * t : 64 + 16 * (t - 2)) : 16 * t; };
    const int am = lane & 15, akb = lane >> 4;
    // the wave's 16-token blocks are 2 mt + wm (mt = 0..3): both halves of a
    // partly filled tile get about the same number of valid blocks
    const uint8_t* a_rd = g_lds + wm * 1024 + (4 * am + (akb ^ chunk_swz(am))) * 16;
    const uint8_t* b_rd = g_lds + kGemmLdsB + rbase * 64 + akb * 4;
    const int b_x = b_swz(rbase) << 4;  // roff(t) is a multiple of 16: same swizzle for every t
    uint32_t s_row[4];                   // the row's scale index at sub-group 0
#pragma unroll
    for (int t = 0; t < 4; ++t) s_row[t] = (uint32_t)tile_row<MODE>(G, rbase + roff(t)) * gpr;
    int s_rd[4];                         // LDS byte offset of the window's first scale of the load
    const int nmt = max(0, min(4, (((G.mvalid + 15) >> 4) - wm + 1) >> 1));  // valid blocks of the wave
    const bf16x8_t k136 = __builtin_bit_cast(bf16x8_t, u32x4_t{0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u});

    f32x4_t acc[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[mt][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // this stage's weight words (as bf16 128 + q) and scales
    auto stage_b = [&](int g, bf16x8_t (&b)[4], float (&sc)[4], uint32_t (&w)[4]) {
        const int b_slot = ((g / kGemmBGroups) & 1) * kGemmSlotB + (((g % kGemmBGroups) << 4) ^ b_x);
        const int s_sub = (g >> RS) - ((kGemmSGroups * (g / kGemmSGroups)) >> RS);  // scale within the load
        const int s_slot = ((g / kGemmSGroups) & 1) * kGemmSlotS + 2 * s_sub;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            w[t] = *reinterpret_cast<const uint32_t*>(b_rd + b_slot + roff(t) * 64);
            sc[t] = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(g_lds + s_rd[t] + s_slot));
        }
        (void)b;
    };
    auto mfma = [](const uint4& a, const bf16x8_t& b, const f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), b, c, 0, 0, 0);
    };

    // Partly filled block set: one block at a time, FMAs right behind.
    auto compute_part = [&](int g, int a_slot) {
        if (nmt == 0) return;
        bf16x8_t b[4];
        float sc[4];
        uint32_t w[4];
        stage_b(g, b, sc, w);
#pragma unroll
        for (int t = 0; t < 4; ++t) b[t] = q4_word_to_bf16x8(w[t]);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            if (mt < nmt) {
                const uint4 ahi = *reinterpret_cast<const uint4*>(a_rd + a_slot + mt * 2048);
                const uint4 alo = LO ? *reinterpret_cast<const uint4*>(a_rd + a_slot + kGemmBM * 64 + mt * 2048) : ahi;
                f32x4_t c0 = mfma(ahi, k136, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f});
                if (LO) c0 = mfma(alo, k136, c0);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    f32x4_t c = mfma(ahi, b[t], c0);
                    if (LO) c = mfma(alo, b[t], c);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[mt][t][i] = __builtin_fmaf(sc[t], c[i], acc[mt][t][i]);
                }
            }
        }
    };

    // All four blocks valid: a software pipeline in which each MFMA is
    // followed by the four scale FMAs of an MFMA that finished long before,
    // so the wave keeps its matrix and vector units busy together.  Block
    // mt's FMAs run behind block mt + 1's MFMAs; block 3's behind the next
    // stage's block 0 (cp / scp carry them).  Per stage:
    //   seed MFMAs of the four blocks, each with a quarter of the nibble
    //   decode behind it; then per block: per n-tile its MFMA(s), then the
    //   lagging block's four FMAs of that n-tile.
    f32x4_t cp[4];
    float scp[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        cp[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        scp[t] = 0.0f;
    }
    auto compute_full = [&](int g, int a_slot) {
        bf16x8_t b[4];
        float sc[4];
        uint32_t w[4];
        stage_b(g, b, sc, w);
        uint4 ahi[4], alo[4];
        f32x4_t c0[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            ahi[mt] = *reinterpret_cast<const uint4*>(a_rd + a_slot + mt * 2048);
            alo[mt] = LO ? *reinterpret_cast<const uint4*>(a_rd + a_slot + kGemmBM * 64 + mt * 2048) : ahi[mt];
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            c0[mt] = mfma(ahi[mt], k136, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f});
            if (LO) c0[mt] = mfma(alo[mt], k136, c0[mt]);
            b[mt] = q4_word_to_bf16x8(w[mt]);
            __builtin_amdgcn_sched_group_barrier(0x008, LO ? 2 : 1, 0);  // seed MFMA(s)
            __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);           // a word's decode
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            f32x4_t cc[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                cc[t] = mfma(ahi[mt], b[t], c0[mt]);
                if (LO) cc[t] = mfma(alo[mt], b[t], cc[t]);
                // the lagging block: mt - 1 of this sub-group, or block 3 of
                // the previous one (with its scales; zeros before the first)
                f32x4_t& dst = acc[mt == 0 ? 3 : mt - 1][t];
                const float sl = mt == 0 ? scp[t] : sc[t];
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[i] = __builtin_fmaf(sl, cp[t][i], dst[i]);
                __builtin_amdgcn_sched_group_barrier(0x008, LO ? 2 : 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) cp[t] = cc[t];
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) scp[t] = sc[t];
    };

    // Stage st (sub-groups g0 = GPS st ..) needs A(st), B(g0 / 4) and
    // scales(g0 / 8).  Everything issued before A(st + 1) is complete once at
    // most OPS_A loads are outstanding (loads complete in issue order and
    // A(st + 1) alone is OPS_A loads), and B / scale loads are issued at
    // least one stage before the A(st + 1) that follows them; after the last
    // A, wait for everything.
    auto stage_begin = [&](int st) {
        const int g = GPS * st;
        if (st + 1 < nst) LP_WAIT_VM_LGKM0(OPS_A);
        else LP_WAIT_VM_LGKM0(0);
        stage_barrier();
        if (st + 2 < nst) issue_a(st + 2, (st + 2) % kGemmASlots);
        if (g % kGemmBGroups == 0 && g + kGemmBGroups < G.ng) issue_b(g / kGemmBGroups + 1, (g / kGemmBGroups + 1) & 1);
        if (g % kGemmSGroups == 0) {
            if (g + kGemmSGroups < G.ng) issue_s(g / kGemmSGroups + 1, (g / kGemmSGroups + 1) & 1);
            const uint32_t first = (uint32_t)(g >> RS);
#pragma unroll
            for (int t = 0; t < 4; ++t)
                s_rd[t] = kGemmLdsS + (rbase + roff(t)) * 32 + 2 * (int)((s_row[t] + first) & 7u);
        }
    };
    issue_a(0, 0);
    issue_b(0, 0);
    issue_s(0, 0);
    if (nst > 1) issue_a(1, 1);
    if (nmt == 4) {
        for (int st = 0; st < nst; ++st) {
            stage_begin(st);
            const int a_slot = (st % kGemmASlots) * kGemmSlotA;
            compute_full(GPS * st, a_slot);
            if (GPS == 2 && GPS * st + 1 < G.ng) compute_full(GPS * st + 1, a_slot + kGemmBM * 64);
        }
        // the last stage's block 3
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[3][t][i] = __builtin_fmaf(scp[t], cp[t][i], acc[3][t][i]);
    } else {
        for (int st = 0; st < nst; ++st) {
            stage_begin(st);
            const int a_slot = (st % kGemmASlots) * kGemmSlotA;
            compute_part(GPS * st, a_slot);
            if (GPS == 2 && GPS * st + 1 < G.ng) compute_part(GPS * st + 1, a_slot + kGemmBM * 64);
        }
    }

    // epilogue: lane holds C rows 4 akb + i (tokens) of column lane & 15 of each tile
    if constexpr (MODE == 0) {
        // act = silu(gate) * up straight into the down GEMM's A image (a.out
        // is the image base; lpk::image_bytes layout, as lp_device.h's
        // write_image_group): the wave's 32 columns n0 + 32 wn .. + 31 are
        // sub-group g of each of its token rows, held by the 16 lanes of one
        // row (column 16 t + am in register t).  Fragment word (d, w) pairs
        // columns 8d + w and 8d + w + 4, so lane am (bit 2 clear) packs its
        // hi part with lane am + 4's (a row shift by 4) and writes the hi
        // word, lane am + 4 the lo word; the seed -136 (sum hi) - 136 (sum
        // lo) comes from a sum over the row's lanes (quad swaps, then the
        // half-row and row mirrors).  All lane exchanges are DPP moves.
        LP_GLOBAL uint8_t* img = gptr_w<uint8_t>(a.out);
        const int g = (G.n0 >> 5) + wn;
        const bool live_g = g < (G.NR >> 5);
        const int ngp = frag_ngp(G.NR);
        const size_t ib = (size_t)image_bytes(G.NR);
        const bool low = (am & 4) == 0;
        const uint32_t part = low ? (uint32_t)g * 64u : (uint32_t)(ngp + g) * 64u;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 16 * (2 * mt + wm) + 4 * akb + i;
                LP_GLOBAL uint8_t* row = img + (size_t)(G.x.p0 + G.m0 + min(m, G.mvalid - 1)) * ib;
                const bool st = m < G.mvalid && live_g;  // the same for lanes am and am ^ 4
                float shi = 0.0f, slo = 0.0f;
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const float gg = acc[mt][t][i], uu = acc[mt][t + 2][i];
                    const float v = gg / (1.0f + expf(-gg)) * uu;
                    const uint32_t h16 = f32_to_bf16_rne(v);
                    const uint32_t l16 = f32_to_bf16_rne(v - bf16_to_f32(h16));
                    shi += bf16_to_f32(h16);
                    slo += bf16_to_f32(l16);
                    // both moves with every lane on (a DPP source lane that is
                    // off reads as zero): pinned here by the empty asm, so that
                    // the select below cannot become a branch around each
                    const int send = (int)(low ? l16 : h16);
                    int up4 = __builtin_amdgcn_mov_dpp(send, 0x104, 0xf, 0xf, true);  // row_shl:4, lane am + 4
                    int dn4 = __builtin_amdgcn_mov_dpp(send, 0x114, 0xf, 0xf, true);  // row_shr:4, lane am - 4
                    asm volatile("" : "+v"(up4), "+v"(dn4));
                    const uint32_t recv = (uint32_t)(low ? up4 : dn4);
                    const uint32_t word = low ? (h16 | (recv << 16)) : (recv | (l16 << 16));
                    const uint32_t off = part + 16u * (uint32_t)(2 * t + (am >> 3)) + 4u * (uint32_t)(am & 3);
                    if (st) *reinterpret_cast<LP_GLOBAL uint32_t*>(row + off) = word;
                }
                shi = row_sum16(shi);
                slo = row_sum16(slo);
                if (st && am == 0)
                    reinterpret_cast<LP_GLOBAL float2*>(row + (size_t)ngp * 128)[g] = make_float2(-136.0f * shi + -136.0f * slo, 0.0f);
            }
        }
    } else {
        float* out = dptr<float>(a.out);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 16 * (2 * mt + wm) + 4 * akb + i;
                if (m >= G.mvalid) continue;
                float* orow = out + (size_t)(G.x.p0 + G.m0 + m) * G.NR;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int r = G.n0 + 64 * wn + 16 * t + am;
                    if (r < G.NR) orow[r] = acc[mt][t][i];
                }
            }
        }
    }
}

template <int MODE, int RS>
__device__ __forceinline__ void gemm_body(const GemmArgs& a) {
    const LayerView& L = a.L;
    const int k = L.top_k;
    // XCD-aware order: workgroup w runs on XCD w % 8, so XCD x takes the
    // contiguous range [x C, x C + C) of the live (tile, row block) items,
    // row blocks innermost: the 128 tokens' A tile and the expert's weight
    // blocks are then fetched into one XCD's L2 and reused there.
    const int count = dptr<const int>(a.W.meta)[2];
    const int live = count * a.nblocks;
    const int C = (live + kXcds - 1) / kXcds;
    const int xcd = blockIdx.x % kXcds, j = blockIdx.x / kXcds;
    const int item = xcd * C + j;
    if (j >= C || item >= live) return;
    const int ti = item / a.nblocks, nb = item - ti * a.nblocks;
    const int tv = dptr<const int>(a.tiles)[ti];
    GemmTile G;
    G.x = load_entry(a.W.et, tv >> 16);
    G.m0 = (tv & 0xffff) * kGemmBM;
    G.mvalid = min(kGemmBM, G.x.ntok - G.m0);
    G.K = MODE == 0 ? L.hidden : L.inter;
    G.NR = MODE == 0 ? L.inter : L.hidden;
    G.ng = G.K >> 5;
    G.ngp = frag_ngp(G.K);
    G.n0 = nb * (MODE == 0 ? kGemmBN / 2 : kGemmBN);
    const int tid = threadIdx.x;
    if (G.x.blob == 0) {  // a routed expert without a slot: flag it, contribute zeros
        if (tid == 0 && nb == 0) atomicOr(dptr<int>(a.W.meta) + 1, kErrMissingExpert);
        if (MODE == 0) {
            // zero act: the tile's two sub-groups of each token row's image
            // (both parts, and the seeds)
            uint8_t* img = dptr<uint8_t>(a.out);
            const int ngp = frag_ngp(G.NR);
            const size_t ib = (size_t)image_bytes(G.NR);
            for (int e = tid; e < G.mvalid * 18; e += blockDim.x) {
                // item (m, sub-group gi, w): w < 8 one 16-byte quarter of
                // part w >> 2, w = 8 the seeds
                const int m = e / 18, q = e - m * 18, gi = q / 9, w = q - gi * 9;
                const int g = (G.n0 >> 5) + gi;
                if (g >= (G.NR >> 5)) continue;
                uint8_t* row = img + (size_t)(G.x.p0 + G.m0 + m) * ib;
                if (w < 8)
                    reinterpret_cast<uint4*>(row + (size_t)((w >> 2) * ngp + g) * 64)[w & 3] = make_uint4(0u, 0u, 0u, 0u);
                else
                    reinterpret_cast<float2*>(row + (size_t)ngp * 128)[g] = make_float2(0.0f, 0.0f);
            }
        } else {
            const int cols = kGemmBN;
            float* out = dptr<float>(a.out);
            for (int e = tid; e < G.mvalid * cols; e += blockDim.x) {
                const int m = e / cols, r = G.n0 + e - m * cols;
                if (r < G.NR) out[(size_t)(G.x.p0 + G.m0 + m) * G.NR + r] = 0.0f;
            }
        }
        return;
    }
    G.off0 = MODE == 0 ? L.gate_off : L.down_off;
    G.off1 = MODE == 0 ? L.up_off : L.down_off;
    const uint64_t ib = (uint64_t)image_bytes(G.K);
    // the tile rows' image addresses (rows past the block repeat its last
    // token) and whether any of them carries a lo part
    int lo = MODE == 1;
    if (tid < kGemmBM) {
        const int pos = G.x.p0 + G.m0 + min(tid, G.mvalid - 1);
        if (MODE == 0) {
            const int tok = dptr<const int>(a.W.perm)[pos] / k;
            reinterpret_cast<uint64_t*>(g_lds + kGemmLdsRows)[tid] = a.a_img + (uint64_t)tok * ib;
            lo = dptr<const int>(a.W.xlo)[tok] != 0;
        } else {
            reinterpret_cast<uint64_t*>(g_lds + kGemmLdsRows)[tid] = a.a_img + (uint64_t)pos * ib;
        }
    }
    if (__syncthreads_or(lo))
        gemm_main<MODE, RS, true>(a, G);
    else
        gemm_main<MODE, RS, false>(a, G);
}

#define LP_BY_RS(group, call)          \
    switch (ilog2_pow2((group) >> 5)) { \
        case 0: call(0); break;         \
        case 1: call(1); break;         \
        default: call(2); break;        \
    }

}  // namespace

// Router logits of a large batch as an MFMA GEMM: logits[t][e] = sum_h
// W[e][h] x[t][h] with W bf16 and x split into three bf16 parts (hi = bf16(x),
// mid = bf16(x - hi), lo = bf16(x - hi - mid): exactly x for normal values),
// so every product is exact and the sums are fp32 in the matrix core (the
// GEMV router's lane order is not kept: its results agree to fp32 rounding).
// The mid and lo MFMAs run only when some lane's x has such a part (never for
// bf16-valued activations).  Grid (ceil(T / 16), ceil(E / 32)), 256 threads:
// the workgroup takes 16 tokens x experts 32 y .. 32 y + 31, wave w the w-th
// quarter of the hidden dimension (its loads four 32-column steps at a time),
// and the four partial tiles meet in LDS, summed in wave order.
extern "C" __global__ void __launch_bounds__(256) lp_gemm_router(const RouteArgs a) {
    __shared__ f32x4_t part[3][2][64];  // waves 1..3: their two partial C tiles per lane
    const int H = a.L.hidden, E = a.L.experts, T = a.T;
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    const int m = lane & 15, kb = lane >> 4;
    const int e0 = blockIdx.y * 32;
    if (e0 >= E) return;  // the whole workgroup
    const int t = min((int)blockIdx.x * 16 + m, T - 1);  // rows past the batch repeat its last token
    const float* xr = dptr<const float>(a.x) + (size_t)t * H + 8 * kb;
    const uint16_t* w0 = dptr<const uint16_t>(a.L.router_w) + (size_t)min(e0 + m, E - 1) * H + 8 * kb;
    const uint16_t* w1 = dptr<const uint16_t>(a.L.router_w) + (size_t)min(e0 + 16 + m, E - 1) * H + 8 * kb;
    f32x4_t c0 = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, c1 = c0;
    auto pack = [](const uint32_t (&q)[8]) {
        return __builtin_bit_cast(bf16x8_t, u32x4_t{q[0] | (q[1] << 16), q[2] | (q[3] << 16),
                                                    q[4] | (q[5] << 16), q[6] | (q[7] << 16)});
    };
    auto step = [&](const float4& xa, const float4& xb, const uint4& wa_, const uint4& wb_) {
        const bf16x8_t wa = __builtin_bit_cast(bf16x8_t, wa_), wb = __builtin_bit_cast(bf16x8_t, wb_);
        const float v[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        uint32_t hi[8], r_any = 0;
        float r[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            hi[i] = f32_to_bf16_rne(v[i]);
            r[i] = v[i] - bf16_to_f32(hi[i]);
            r_any |= __float_as_uint(r[i]) << 1;  // ignore the sign of zero
        }
        const bf16x8_t ah = pack(hi);
        c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, wa, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, wb, c1, 0, 0, 0);
        if (__ballot(r_any != 0u)) {
            uint32_t mid[8], lo[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                mid[i] = f32_to_bf16_rne(r[i]);
                lo[i] = f32_to_bf16_rne(r[i] - bf16_to_f32(mid[i]));
            }
            const bf16x8_t am = pack(mid), al = pack(lo);
            c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, wa, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, wb, c1, 0, 0, 0);
            c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, wa, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, wb, c1, 0, 0, 0);
        }
    };
    // this wave's quarter of the 32-column steps (H is a multiple of 32),
    // four steps' loads in flight before their MFMAs
    const int ns = H >> 5;
    const int hend = 32 * ((ns * (wave + 1)) >> 2);
    int h = 32 * ((ns * wave) >> 2);
    for (; h + 128 <= hend; h += 128) {
        float4 xa[4], xb[4];
        uint4 wa[4], wb[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            xa[q] = *reinterpret_cast<const float4*>(xr + h + 32 * q);
            xb[q] = *reinterpret_cast<const float4*>(xr + h + 32 * q + 4);
            wa[q] = *reinterpret_cast<const uint4*>(w0 + h + 32 * q);
            wb[q] = *reinterpret_cast<const uint4*>(w1 + h + 32 * q);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) step(xa[q], xb[q], wa[q], wb[q]);
    }
    for (; h < hend; h += 32)
        step(*reinterpret_cast<const float4*>(xr + h), *reinterpret_cast<const float4*>(xr + h + 4),
             *reinterpret_cast<const uint4*>(w0 + h), *reinterpret_cast<const uint4*>(w1 + h));
    if (wave > 0) {
        part[wave - 1][0][lane] = c0;
        part[wave - 1][1][lane] = c1;
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < 3; ++w) {
        c0 += part[w][0][lane];
        c1 += part[w][1][lane];
    }
    // lane holds C rows 4 kb + i (tokens) of column m (experts e0 + m, e0 + 16 + m)
    float* logits = dptr<float>(a.W.logits);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int tt = (int)blockIdx.x * 16 + 4 * kb + i;
        if (tt >= T) continue;
        if (e0 + m < E) logits[(size_t)tt * E + e0 + m] = c0[i];
        if (e0 + 16 + m < E) logits[(size_t)tt * E + e0 + 16 + m] = c1[i];
    }
}

// The tile list: for each routed expert u < meta[0], ceil(ntok / kGemmBM)
// token blocks, as (u << 16) | block; meta[2] = the count.  One workgroup.
extern "C" __global__ void __launch_bounds__(256) lp_gemm_tiles(const GemmArgs a) {
    __shared__ int sh[4];
    const int nu = dptr<const int>(a.W.meta)[0];
    const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    int* tiles = dptr<int>(a.tiles);
    int base = 0;
    for (int u0 = 0; u0 < nu; u0 += 256) {
        const int u = u0 + tid;
        const int nb = u < nu ? (load_entry(a.W.et, u).ntok + kGemmBM - 1) / kGemmBM : 0;
        int x = nb;  // inclusive scan over the workgroup
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(x, o, 64);
            if (lane >= o) x += y;
        }
        if (lane == 63) sh[wave] = x;
        __syncthreads();
        int wb = 0, tot = 0;
        for (int w = 0; w < 4; ++w) {
            wb += w < wave ? sh[w] : 0;
            tot += sh[w];
        }
        const int first = base + wb + x - nb;
        for (int b = 0; b < nb; ++b)
            if (first + b < a.max_tiles) tiles[first + b] = (u << 16) | b;
        base += tot;
        __syncthreads();
    }
    if (tid == 0) dptr<int>(a.W.meta)[2] = min(base, a.max_tiles);
}

extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) lp_gemm_gateup(const GemmArgs a) {
#define LP_G(rs) gemm_body<0, rs>(a)
    LP_BY_RS(a.L.group, LP_G)
#undef LP_G
}

extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) lp_gemm_down(const GemmArgs a) {
#define LP_G(rs) gemm_body<1, rs>(a)
    LP_BY_RS(a.L.group, LP_G)
#undef LP_G
}
