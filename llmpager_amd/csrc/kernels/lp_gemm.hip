// Prefill: the grouped expert projections as MFMA GEMMs over the dispatch
// tables (the reference prefills with one GEMV per token, decode.rs:469-531;
// the arithmetic each output restates is q4g64.cu:19-81's).
//
// A tile is (routed expert, block of kGemmBM = 128 of its tokens, block of
// kGemmBN = 256 weight rows), eight waves; wave w owns 32 rows (two 16-row
// MFMA tiles) against all 128 tokens (eight 16-token tiles), so every weight
// is dequantised once per tile.  Gate/up tiles take 128 act columns: wave w's
// gate rows and the same up rows, so SiLU * up is the epilogue.
//
// The MFMA is v_mfma_f32_16x16x32_f16 with the weights as its first operand
// and the tokens as its second: C[row][token], fp32 accumulation over all of
// K.  Weights: each lane turns a q4 word into fp16 (q - 8) s with two packed
// fp16 operations per two values (1024 + q by the 0x6400 exponent trick,
// minus 1032, exact; times the group's fp16 scale, one rounding).  Tokens:
// fp16 images of x (gate/up, through the dispatch permutation) or of act
// (down), each row scaled by a power of two (lp_device.h's h16_exp).
//
// K runs in stages of 64 columns (two sub-groups).  Per stage, direct-to-LDS
// loads (no registers, no LDS stores) bring 128 bytes of each token row and 32
// bytes of each weight row into one of kGemmSlots slots, three stages ahead;
// every fourth stage a 16-scale window of each row.  Within a stage lane (r,
// kb) of an MFMA takes sub-group kb >> 1, words 2 (kb & 1) + j at step j, on
// both operands.
//
// act leaves gate/up as fp16 images with one exponent per (row, 128 columns),
// the tile's own maximum; the down GEMM rescales each staged chunk in LDS to
// the row's largest exponent before its MFMAs and scales y back.
#include <type_traits>

#include "lp_device.h"

using namespace lp;
using namespace lpk;

namespace {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

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

__device__ __forceinline__ void dma16(uint64_t base, uint32_t off, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}

// LDS address of g_lds (the M0 operand of the direct loads is an LDS address).
__device__ __forceinline__ uint32_t lds_base() {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)g_lds;
}

// Wait until at most n vector-memory loads of this wave are outstanding and
// its LDS reads are done; with the loads completing in issue order this is
// "every load issued before the last n has landed".
#define LP_WAIT_VM_LGKM0(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4))

// s_barrier as a compiler-level memory fence too: no LDS access or load moves
// across it.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Token n's (n = tile token mod 16) 16-byte word c of a stage sits at
// position c ^ tok_swz(n) of its 128-byte LDS row: an MFMA operand read (16
// tokens, one word each) then touches 16 distinct 16-byte bank groups of 256
// bytes, and 8 distinct of 128 bytes per 8 lanes.
__device__ __forceinline__ int tok_swz(int n) { return (n ^ (n >> 3)) & 7; }

// Weight row rho's two 16-byte sub-group pieces of a stage: piece h at
// position h ^ w_swz(rho) (rows 8 apart then differ in their 8-byte reads).
__device__ __forceinline__ int w_swz(int rho) { return (rho >> 3) & 1; }

// The act column (0..15 within a wave's 16) of MFMA row r of a gate/up tile:
// lane group kb of the C tile holds rows 4 kb .. 4 kb + 3, which are then the
// columns of half kb & 1 of the image's word kb >> 1, in image order.
__device__ __forceinline__ int act_col(int r) {
    const int q = r >> 2, i = r & 3;
    return 8 * (q >> 1) + 2 * (q & 1) + ((i & 1) << 2) + (i >> 1);
}

// A q4 word (8 values, nibble v of byte v / 2, low first) as fp16 (q - 8) s in
// image order (0, 4, 1, 5, 2, 6, 3, 7): 1024 + q exactly from the exponent
// trick, minus 1032 exactly, times s with one rounding.
__device__ __forceinline__ f16x8_t q4_word_to_f16x8(uint32_t b, f16x2_t s) {
    const f16x2_t bias = {(_Float16)1032.0f, (_Float16)1032.0f};
    const f16x2_t h0 = (__builtin_bit_cast(f16x2_t, and_or(b, 0x000F000Fu, 0x64006400u)) - bias) * s;
    const f16x2_t h1 = (__builtin_bit_cast(f16x2_t, and_or(b >> 4, 0x000F000Fu, 0x64006400u)) - bias) * s;
    const f16x2_t h2 = (__builtin_bit_cast(f16x2_t, and_or(b >> 8, 0x000F000Fu, 0x64006400u)) - bias) * s;
    const f16x2_t h3 = (__builtin_bit_cast(f16x2_t, and_or(b >> 12, 0x000F000Fu, 0x64006400u)) - bias) * s;
    return f16x8_t{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

// A value the whole wave holds, as a scalar (so that branches on it stay
// scalar branches).
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// 2^d as fp16 bits for d in [-127, 0] (0 below 2^-24).
__device__ __forceinline__ uint32_t f16_pow2(int d) {
    return d >= -14 ? (uint32_t)(d + 15) << 10 : d >= -24 ? 1u << (d + 24) : 0u;
}

// Waves per tile and the copies each issues per stage: RT MFMA row tiles
// (16 rows each) per wave; tokens in copies of 8 rows x 128 B, weights and
// scale windows in copies of 32 rows x 32 B.
constexpr int RT = kGemmRowTiles;
constexpr int kWaves = kGemmWaves;
constexpr int NTD = kGemmBM / kWaves / 8;  // token copies per wave per stage
constexpr int NWD = 16 * RT / 32;          // weight (and scale) copies per wave per stage
static_assert(kWaves * 16 * RT == kGemmBN && NTD >= 1 && NWD >= 1, "GEMM tile shape");

template <int MODE, int RS>
__device__ __forceinline__ void gemm_body(const GemmArgs& a) {
    const LayerView& L = a.L;
    // XCD-aware order: workgroup w runs on XCD w % 8, so XCD x takes the
    // contiguous range [x C, x C + C) of the live (tile, row block) items,
    // row blocks innermost: the 128 tokens' images and the expert's weight
    // rows are then fetched into one XCD's L2 and reused there.
    const int count = uni(dptr<const int>(a.W.meta)[2]);
    const int live = count * a.nblocks;
    const int C = (live + kXcds - 1) / kXcds;
    const int xcd = blockIdx.x % kXcds, jx = blockIdx.x / kXcds;
    const int item = xcd * C + jx;
    if (jx >= C || item >= live) return;
    const int ti = item / a.nblocks, nb = item - ti * a.nblocks;
    const int tv = uni(dptr<const int>(a.tiles)[ti]);
    ExpertEntry x = load_entry(a.W.et, tv >> 16);
    x.p0 = uni(x.p0);
    x.ntok = uni(x.ntok);
    const int m0 = (tv & 0xffff) * kGemmBM;
    const int mvalid = min(kGemmBM, x.ntok - m0);
    const int K = MODE == 0 ? L.hidden : L.inter;
    const int NR = MODE == 0 ? L.inter : L.hidden;
    const int ng = K >> 5, nst = frag_ngp(K) >> 1;
    const int gpr = ng >> RS;                         // scales per weight row
    const int nch = act_chunks(L.inter);
    const int n0 = nb * (MODE == 0 ? kActChunk : kGemmBN);  // gate/up: first act column; down: first row
    const uint32_t rowbytes = (uint32_t)himage_bytes(K);
    const int tid = threadIdx.x, lane = lane_id();
    const int wave = uni(tid >> 6);  // uniform: DMA targets stay scalar
    int* meta = dptr<int>(a.W.meta);
    if (x.blob == 0) {  // a routed expert without a slot: flag it, contribute zeros
        if (tid == 0 && nb == 0) atomicOr(meta + 1, kErrMissingExpert);
        if (MODE == 0) {
            // the tile's four sub-groups of each token's act image (256
            // contiguous bytes) and its chunk exponent
            uint8_t* img = dptr<uint8_t>(a.out);
            const size_t ob = (size_t)himage_bytes(NR);
            for (int e = tid; e < mvalid * 16; e += blockDim.x) {
                const int m = e >> 4, q = e & 15;
                reinterpret_cast<uint4*>(img + (size_t)(x.p0 + m0 + m) * ob + (size_t)(n0 >> 5) * 64)[q] =
                    make_uint4(0u, 0u, 0u, 0u);
            }
            for (int m = tid; m < mvalid; m += blockDim.x)
                dptr<int>(a.W.act)[(size_t)(x.p0 + m0 + m) * nch + nb] = kExpNone;
        } else {
            float* out = dptr<float>(a.out);
            for (int e = tid; e < mvalid * kGemmBN; e += blockDim.x) {
                const int m = e / kGemmBN, r = n0 + e - m * kGemmBN;
                if (r < NR) out[(size_t)(x.p0 + m0 + m) * NR + r] = 0.0f;
            }
        }
        return;
    }

    // --- the tile's token rows: image offsets, exponents (down: per-chunk shifts) ---
    uint32_t* rows_l = reinterpret_cast<uint32_t*>(g_lds + kGemmLdsRows);
    int* exp_l = reinterpret_cast<int*>(g_lds + kGemmLdsExp);
    int8_t* shift_l = reinterpret_cast<int8_t*>(g_lds + kGemmLdsShift);
    if (tid < kGemmBM) {
        // rows past the block repeat its last token
        const int pos = x.p0 + m0 + min(tid, mvalid - 1);
        if (MODE == 0) {
            const int tok = dptr<const int>(a.W.perm)[pos] / L.top_k;
            rows_l[tid] = (uint32_t)tok * rowbytes;
            exp_l[tid] = dptr<const int>(a.W.xexp)[tok];
        } else {
            rows_l[tid] = (uint32_t)pos * rowbytes;
            const int* ae = dptr<const int>(a.W.act) + (size_t)pos * nch;
            int mx = kExpNone;
            for (int c = 0; c < nch; ++c) mx = max(mx, ae[c]);
            for (int c = 0; c < nch; ++c) shift_l[tid * kGemmMaxChunks + c] = (int8_t)max(ae[c] - mx, -127);
            exp_l[tid] = mx;
        }
    }
    __syncthreads();

    // --- rows: wave w owns the tile's weight rows 16 RT w .. 16 RT (w + 1) -
    // 1, MFMA row tiles t = 0 .. RT - 1 (row 16 t + r).  Gate/up: the wave's
    // 8 RT act columns n0 + 8 RT w .. in gate tiles 0 .. RT / 2 - 1 and the
    // same in up tiles RT / 2 .. RT - 1 ---
    constexpr int RH = RT / 2;
    auto mat_row = [&](int t, int r) {
        return min(MODE == 0 ? n0 + 8 * RT * wave + 16 * (t % RH) + act_col(r) : n0 + 16 * RT * wave + 16 * t + r,
                   NR - 1);
    };
    auto region = [&](int t) { return (uint32_t)(MODE == 0 ? (t >= RH ? L.up_off : L.gate_off) : L.down_off); };
    const uint32_t sbytes = (uint32_t)NR * (uint32_t)gpr * 2u;

    // --- load side: a uniform 64-bit base plus per-lane 32-bit offsets ---
    const uint32_t lds0 = lds_base();
    const uint64_t a_base = a.a_img;
    const uint64_t w_base = (uint64_t)(uint32_t)uni((int)(uint32_t)x.blob) | ((uint64_t)(uint32_t)uni((int)(uint32_t)(x.blob >> 32)) << 32);
    // tokens: copy u of the wave takes tile tokens 8 (NTD w + u) + (l >> 3),
    // lane l filling position l & 7 of its row (word (l & 7) ^ tok_swz); every
    // wave issues all its copies (rows past the block repeat its last token),
    // so the main loop's wait counts are constants
    uint32_t t_off[NTD];
#pragma unroll
    for (int u = 0; u < NTD; ++u) {
        const int tt = 8 * (NTD * wave + u) + (lane >> 3);
        t_off[u] = rows_l[tt] + (uint32_t)(((lane & 7) ^ tok_swz(tt & 15)) * 16);
    }
    // weights and scale windows: copy u of the wave fills LDS rows 16 RT w +
    // 32 u + (l >> 1) (tile 2 u + (l >> 5), row (l >> 1) & 15), lane l piece
    // l & 1 (weights: sub-group 2 st + ((l & 1) ^ w_swz); scales: half l & 1
    // of the 16-scale window)
    const int d_r = (lane >> 1) & 15;
    const int d_h = (lane & 1) ^ w_swz(d_r);
    uint32_t w_row[NWD], s_row[NWD], s_reg[NWD];
#pragma unroll
    for (int u = 0; u < NWD; ++u) {
        const int t = 2 * u + (lane >> 5);
        w_row[u] = region(t) + sbytes + (uint32_t)mat_row(t, d_r) * (uint32_t)ng * 16u;
        s_row[u] = (uint32_t)mat_row(t, d_r) * (uint32_t)gpr;  // the row's first scale
        s_reg[u] = region(t) + 16u * (uint32_t)(lane & 1);
    }

    // Pipeline step i issues the token rows of stage i + 3 (NTD loads) and
    // the weight rows of stage i + 4 (NWD, plus NWD for the scale window of
    // stages i + 4 .. i + 7 when i + 4 is a multiple of 4): weights run one
    // stage ahead of the tokens, so that stage st's MFMAs share the wave
    // with the decode of stage st + 1's weights.  Slots are compile-time
    // (stage % 4).
    auto issue_tok = [&](auto slot_c, int st) {
        constexpr int SLOT = decltype(slot_c)::value;
        const uint64_t base = a_base + (uint64_t)st * 128;
#pragma unroll
        for (int u = 0; u < NTD; ++u) dma16(base, t_off[u], lds0 + SLOT * kGemmSlotT + 8 * (NTD * wave + u) * 128);
    };
    auto issue_w = [&](auto slot_c, int st) {
        constexpr int SLOT = decltype(slot_c)::value;
        const uint32_t sg = (uint32_t)min(2 * st + d_h, ng - 1);
#pragma unroll
        for (int u = 0; u < NWD; ++u)
            dma16(w_base, w_row[u] + sg * 16u, lds0 + kGemmLdsW + SLOT * kGemmSlotW + (NWD * wave + u) * 1024);
        if constexpr (SLOT == 0) {
            // the window starts at the 8-aligned scale index at or below the
            // row's first scale of stages st .. st + 3: 16 scales cover them
            const int q = st >> 2;
#pragma unroll
            for (int u = 0; u < NWD; ++u) {
                const uint32_t c0 = (s_row[u] + (uint32_t)((8 * q) >> RS)) & ~7u;
                dma16(w_base, s_reg[u] + c0 * 2u, lds0 + kGemmLdsS + (q & 1) * kGemmSlotS + (NWD * wave + u) * 1024);
            }
        }
    };

    // --- read side: lane (r, kb) of the MFMAs ---
    const int r = lane & 15, kb = lane >> 4;
    int t_rd[2];  // token r's word 2 kb + j of a stage
#pragma unroll
    for (int j = 0; j < 2; ++j) t_rd[j] = r * 128 + (((2 * kb + j) ^ tok_swz(r)) * 16);
    int w_rd[RT], s_rd[RT];
    uint32_t rsb[RT];  // the row's first scale index
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        const int rho = 16 * RT * wave + 16 * t + r;
        w_rd[t] = rho * 32 + (((kb >> 1) ^ w_swz(rho)) * 16) + 8 * (kb & 1);
        s_rd[t] = rho * 32;
        rsb[t] = (uint32_t)mat_row(t, r) * (uint32_t)gpr;
    }
    // valid 16-token tiles, rounded up to even (the loop comes in four
    // unrolled forms; a tile past the block computes on stale rows, unstored)
    const int nmt2 = min(8, (((mvalid + 15) >> 4) + 1) & ~1);

    f32x4_t acc[RT][8];
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) acc[t][mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // Stage st's weight words and scale bits (LDS) of the lane's RT row
    // tiles (SLOT = st % 4); decode turns them into the MFMA operands
    // (wd[j][t]: step j, row tile t), zero past the last sub-group.  Within a
    // window the lane's scale sits at ((rsb + 8 q >> RS) & 7) + ((2 (st % 4) +
    // (kb >> 1)) >> RS).
    auto read_w = [&](auto slot_c, int st, uint2 (&wv)[RT], uint32_t (&sv)[RT]) {
        constexpr int SLOT = decltype(slot_c)::value;
        const uint8_t* wb = g_lds + kGemmLdsW + SLOT * kGemmSlotW;
        const int q = st >> 2;
        const uint8_t* sb = g_lds + kGemmLdsS + (q & 1) * kGemmSlotS;
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            wv[t] = *reinterpret_cast<const uint2*>(wb + w_rd[t]);
            const uint32_t pos = ((rsb[t] + (uint32_t)((8 * q) >> RS)) & 7u) + (uint32_t)((2 * SLOT + (kb >> 1)) >> RS);
            sv[t] = *reinterpret_cast<const uint16_t*>(sb + s_rd[t] + 2 * pos);
        }
    };
    auto decode = [&](int st, const uint2 (&wv)[RT], const uint32_t (&sv)[RT], f16x8_t (&wd)[2][RT]) {
        const bool live = 2 * st + (kb >> 1) < ng;
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint32_t sb = live ? sv[t] : 0u;
            const f16x2_t sc = __builtin_bit_cast(f16x2_t, sb | (sb << 16));
            wd[0][t] = q4_word_to_f16x8(wv[t].x, sc);
            wd[1][t] = q4_word_to_f16x8(wv[t].y, sc);
        }
    };

    // Stage st's MFMAs (slot SLOT) with stage st + 1's weights read and
    // decoded between them (wd: stage st's decoded weights in, stage st + 1's
    // out; past the last stage the decode reads a stale slot, unused).
    auto compute = [&](auto nm_c, auto slot_c, int st, f16x8_t (&wd)[2][RT]) {
        constexpr int NM = decltype(nm_c)::value;
        constexpr int SLOT = decltype(slot_c)::value;
        const uint8_t* tb = g_lds + SLOT * kGemmSlotT;
        // the next stage's weight reads first: its decode waits on them
        uint2 wv[RT];
        uint32_t sv[RT];
        read_w(std::integral_constant<int, (SLOT + 1) & 3>{}, st + 1, wv, sv);
        __builtin_amdgcn_sched_barrier(0);
        uint4 bt[2][NM];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) bt[j][mt] = *reinterpret_cast<const uint4*>(tb + mt * 2048 + t_rd[j]);
        f16x8_t wn[2][RT];
        decode(st + 1, wv, sv, wn);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) {
                const f16x8_t b = __builtin_bit_cast(f16x8_t, bt[j][mt]);
#pragma unroll
                for (int t = 0; t < RT; ++t)
                    acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wd[j][t], b, acc[t][mt], 0, 0, 0);
            }
        // order: the token reads, then each MFMA followed by (at most) two
        // vector instructions of the next stage's decode
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * NM, 0);
#pragma unroll
        for (int i = 0; i < 2 * RT * NM; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int t = 0; t < RT; ++t) wd[j][t] = wn[j][t];
    };

    // down: stage st's act chunk in LDS times 2^(chunk exponent - row
    // exponent), 128 / TPT bytes of one token per thread
    constexpr int TPT = 64 * kWaves / kGemmBM;  // threads per token
    auto rescale = [&](auto slot_c, int st) {
        constexpr int SLOT = decltype(slot_c)::value;
        const int tt = tid / TPT;
        const int d = shift_l[tt * kGemmMaxChunks + (st >> 1)];
        if (tt >= mvalid || d == 0) return;
        const uint32_t f = f16_pow2(d);
        const f16x2_t f2 = __builtin_bit_cast(f16x2_t, f | (f << 16));
        uint4* p = reinterpret_cast<uint4*>(g_lds + SLOT * kGemmSlotT + tt * 128 + (tid % TPT) * (128 / TPT));
#pragma unroll
        for (int h = 0; h < 8 / TPT; ++h) {
            uint4 v = p[h];
            v.x = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, v.x) * f2);
            v.y = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, v.y) * f2);
            v.z = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, v.z) * f2);
            v.w = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, v.w) * f2);
            p[h] = v;
        }
    };

    // Token rows of stage st sit in slot st % 4, its weight rows too, its
    // scale window in window slot (st / 4) % 2.  Loads complete in issue
    // order, so "step i's loads have landed" is "at most the loads of the
    // steps after it are outstanding": step i issues NTD + NWD loads, NWD more
    // when i is a multiple of 4, while i + 4 < nst.  Main-loop step st (after
    // the barrier that puts every wave past stage st - 1, whose slots it
    // refills) needs stage st's tokens and stage st + 1's weights, i.e. step
    // st - 3, so steps st - 2 and st - 1 may stay outstanding.  Down also
    // rescales stage st + 1's tokens during step st, so it waits for those
    // (step st - 2's token loads); the next barrier publishes the rescale.
    // The last three steps wait for everything.
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    auto step = [&](auto nm_c, auto slot_c, int st, f16x8_t (&wd)[2][RT]) {
        constexpr int U = decltype(slot_c)::value;
        constexpr int OUT = (MODE == 0 ? 2 * (NTD + NWD) : NTD + 2 * NWD) + NWD * ((U == 1) + (U == 2));
        if (st + 3 < nst) {
            LP_WAIT_VM_LGKM0(OUT);
        } else {
            LP_WAIT_VM_LGKM0(0);
        }
        stage_barrier();
        if (st + 3 < nst) issue_tok(std::integral_constant<int, (U + 3) & 3>{}, st + 3);
        if (st + 4 < nst) issue_w(slot_c, st + 4);
        if (MODE == 1 && st + 1 < nst) rescale(std::integral_constant<int, (U + 1) & 3>{}, st + 1);
        compute(nm_c, slot_c, st, wd);
    };
    auto run = [&](auto nm_c) {
        // steps -4 .. -1 (weights of stage 0 with its window: 2 NWD loads;
        // then per stage NTD token loads and NWD weight loads)
        issue_w(I0{}, 0);
        issue_tok(I0{}, 0);
        if (nst > 1) issue_w(I1{}, 1);
        if (nst > 1) issue_tok(I1{}, 1);
        if (nst > 2) issue_w(I2{}, 2);
        if (nst > 2) issue_tok(I2{}, 2);
        if (nst > 3) issue_w(I3{}, 3);
        f16x8_t wd[2][RT];
        {
            // stage 0's weights (step -4) and, for down, its tokens (step -3)
            if (nst > 3) {
                LP_WAIT_VM_LGKM0(MODE == 0 ? 3 * (NTD + NWD) : 3 * NWD + 2 * NTD);
            } else {
                LP_WAIT_VM_LGKM0(0);
            }
            stage_barrier();
            uint2 wv[RT];
            uint32_t sv[RT];
            read_w(I0{}, 0, wv, sv);
            decode(0, wv, sv, wd);
            if (MODE == 1) rescale(I0{}, 0);
        }
        int st = 0;
        for (; st + 4 <= nst; st += 4) {
            step(nm_c, I0{}, st, wd);
            step(nm_c, I1{}, st + 1, wd);
            step(nm_c, I2{}, st + 2, wd);
            step(nm_c, I3{}, st + 3, wd);
        }
        if (st < nst) step(nm_c, I0{}, st, wd);
        if (st + 1 < nst) step(nm_c, I1{}, st + 1, wd);
        if (st + 2 < nst) step(nm_c, I2{}, st + 2, wd);
    };
    switch (nmt2) {
        case 2: run(std::integral_constant<int, 2>{}); break;
        case 4: run(std::integral_constant<int, 4>{}); break;
        case 6: run(std::integral_constant<int, 6>{}); break;
        default: run(std::integral_constant<int, 8>{}); break;
    }

    // --- epilogues: lane (r, kb) holds C rows 4 kb + i of token 16 mt + r ---
    if constexpr (MODE == 0) {
        // act = silu(gate) * up at the x rows' scale (gate tile h with up tile
        // h + RT / 2: act columns n0 + 8 RT w + 16 h + act_col(4 kb + i)); the
        // tile's 128 columns of each token get the exponent of their largest
        // magnitude (over the four lane groups, then the waves through LDS,
        // reusing the token slots), then go out as fp16 image words: lane
        // group kb's four columns of tile h are half kb & 1 of word kb >> 1 of
        // the 16 columns from column c = n0 + 8 RT w + 16 h, i.e. at byte 64
        // (c / 32) + 2 (c % 32) + 8 kb of the row.
        const int I = NR;
        __syncthreads();
        float* red = reinterpret_cast<float*>(g_lds);  // [128 tokens][kWaves]
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) {
            const int tt = 16 * mt + r;
            const int ex = exp_l[tt];
            float m = 0.0f;
#pragma unroll
            for (int h = 0; h < RH; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int col = n0 + 8 * RT * wave + 16 * h + act_col(4 * kb + i);
                    const float g = __builtin_ldexpf(acc[h][mt][i], ex), u = __builtin_ldexpf(acc[h + RH][mt][i], ex);
                    // silu with the hardware exp2 and reciprocal: a few ulp
                    // of fp32, far below the fp16 rounding that follows
                    const float e = __builtin_amdgcn_exp2f(-1.44269504f * g);
                    const float v = col < I ? g * __builtin_amdgcn_rcpf(1.0f + e) * u : 0.0f;
                    acc[h][mt][i] = v;
                    m = fmaxf(m, fabsf(v));
                }
            m = fmaxf(m, __shfl_xor(m, 16, 64));
            m = fmaxf(m, __shfl_xor(m, 32, 64));
            if (kb == 0) red[tt * kWaves + wave] = m;
        }
        __syncthreads();
        uint8_t* img = dptr<uint8_t>(a.out);
        const size_t ob = (size_t)himage_bytes(I);
        auto woff = [&](int h) {
            const int c = n0 + 8 * RT * wave + 16 * h;
            return (uint32_t)(c >> 5) * 64u + 2u * (uint32_t)(c & 31) + 8u * (uint32_t)kb;
        };
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) {
            const int tt = 16 * mt + r;
            if (tt >= mvalid) continue;
            float M = 0.0f;
#pragma unroll
            for (int w4 = 0; w4 < kWaves; w4 += 4) {
                const float4 rv = *reinterpret_cast<const float4*>(red + tt * kWaves + w4);
                M = fmaxf(M, fmaxf(fmaxf(rv.x, rv.y), fmaxf(rv.z, rv.w)));
            }
            const int ae = M > 0.0f ? h16_exp(M) : kExpNone;
            const int p = x.p0 + m0 + tt;
#pragma unroll
            for (int h = 0; h < RH; ++h) {
                uint32_t hv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    hv[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)__builtin_ldexpf(acc[h][mt][i], -ae));
                *reinterpret_cast<uint2*>(img + (size_t)p * ob + woff(h)) =
                    make_uint2(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16));
            }
            if (wave == 0 && kb == 0) dptr<int>(a.W.act)[(size_t)p * nch + nb] = ae;
        }
    } else {
        float* out = dptr<float>(a.out);
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) {
            const int tt = 16 * mt + r;
            if (tt >= mvalid) continue;
            const int ex = exp_l[tt];
            float* orow = out + (size_t)(x.p0 + m0 + tt) * NR;
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                const int row = n0 + 16 * RT * wave + 16 * t + 4 * kb;
                if (row < NR)
                    *reinterpret_cast<float4*>(orow + row) =
                        make_float4(__builtin_ldexpf(acc[t][mt][0], ex), __builtin_ldexpf(acc[t][mt][1], ex),
                                    __builtin_ldexpf(acc[t][mt][2], ex), __builtin_ldexpf(acc[t][mt][3], ex));
            }
        }
    }
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
        const int x = wave_incl_scan(nb);  // inclusive scan over the workgroup
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

extern "C" __global__ void __launch_bounds__(64 * kGemmWaves) lp_gemm_gateup(const GemmArgs a) {
#define LP_G(rs) gemm_body<0, rs>(a)
    LP_BY_RS(a.L.group, LP_G)
#undef LP_G
}

extern "C" __global__ void __launch_bounds__(64 * kGemmWaves) lp_gemm_down(const GemmArgs a) {
#define LP_G(rs) gemm_body<1, rs>(a)
    LP_BY_RS(a.L.group, LP_G)
#undef LP_G
}
