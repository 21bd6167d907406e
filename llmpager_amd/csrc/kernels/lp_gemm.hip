// Prefill: the grouped expert projections as MFMA GEMMs over the dispatch
// tables (the reference prefills with one GEMV per token, decode.rs:469-531;
// the arithmetic each output restates is q4g64.cu:19-81's).
//
// A tile is (routed expert, block of kGemmBM of its tokens, block of weight
// rows): gate/up tiles take 64 rows of gate and the same 64 rows of up so
// that SiLU * up is the epilogue; down tiles take 128 rows.  K runs over
// 32-column sub-groups, one pipeline stage each:
//   A (activations): the token rows' fragment images (bf16 hi = bf16(x), lo =
//     bf16(x - hi), MFMA operand order, and the -136 * part sums), gathered
//     through the dispatch permutation;
//   B (weights): the q4 nibbles of the stage, turned into bf16 128 + q once
//     per stage by the loading threads (v_bitop3_b32 per word pair) for all
//     four waves, plus the rows' f16 scales as f32;
//   v_mfma_f32_16x16x32_bf16 over one sub-group is then sum_k (hi + lo)_k *
//     (128 + q_k), seeded with -136 * sum_k (hi + lo)_k so it equals
//     sum_k x_k (q_k - 8) exactly up to fp32 rounding, and the sub-group's
//     scale is applied in fp32.  A stage whose lo parts are all zero (bf16
//     activations) skips the lo MFMAs.
// Stage g + 1's loads are issued (unconditionally, the last one repeated)
// before stage g's MFMAs, into registers, and written to the other LDS
// buffer after them.
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

// One matrix (a q4 region of `rows` x `cols`) read through a raw buffer
// resource: loads past the region return zero.
struct Region {
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t data;  // byte offset of the nibbles
    int ng, gpr;    // 32-column sub-groups per row, scales per row
};

__device__ __forceinline__ Region region_at(uint64_t base, int rows, int cols, int rs) {
    Region r;
    r.ng = cols >> 5;
    r.gpr = r.ng >> rs;
    const uint32_t sbytes = (uint32_t)rows * r.gpr * 2;
    r.data = sbytes;
    r.rsrc = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(base), (short)0,
                                               (int)(sbytes + (uint32_t)rows * r.ng * 16), kBufferWord3);
    return r;
}

struct StageRegs {
    uint4 a0, a1;     // this thread's two A units
    uint4 q;          // waves 0-1: one weight row's 32 nibbles
    uint32_t sc;      // waves 2-3: one row's f16 scale bits
    float seed;       // waves 2-3: one (part, token) seed
};

// Issue stage g's loads.  Thread t: A units t and t + 256 (part = u >> 8,
// token = (u >> 2) & 63, 16-byte unit u & 3); waves 0-1: weight row t's
// nibbles; waves 2-3: row (t - 128)'s scale and seed (t - 128).
template <int MODE, int RS>
__device__ __forceinline__ void stage_load(StageRegs& R, const uint64_t* rowimg, const Region& r0,
                                           const Region& r1, int n0, int ngp, int g) {
    const int t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: the descriptors stay scalar
    const int u0 = t, u1 = t + 256;
    R.a0 = gptr<uint4>(rowimg[(u0 >> 2) & 63] + (uint64_t)(u0 >> 8) * ngp * 64 + (uint64_t)g * 64)[u0 & 3];
    R.a1 = gptr<uint4>(rowimg[(u1 >> 2) & 63] + (uint64_t)(u1 >> 8) * ngp * 64 + (uint64_t)g * 64)[u1 & 3];
    // gate/up: odd waves take the up matrix (rows 64-127 of the tile are the
    // same matrix rows as 0-63); down: one matrix, 128 rows
    const bool up = MODE == 0 && (wave & 1);
    const __amdgpu_buffer_rsrc_t rsrc = up ? r1.rsrc : r0.rsrc;
    const int i = t & 127;
    const int row = n0 + (MODE == 0 ? (i & 63) : i);
    if (wave < 2) {  // waves 0-1: row i's nibbles
        R.q = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)(r0.data + ((uint32_t)row * r0.ng + g) * 16u), 0, 0));
    } else {  // waves 2-3: row i's scale, seed i
        R.sc = __builtin_amdgcn_raw_buffer_load_b16(rsrc, (int)(((uint32_t)row * r0.gpr + (g >> RS)) * 2u), 0, 0);
        R.seed = gptr<float>(rowimg[i & 63] + (uint64_t)ngp * 128)[2 * g + (i >> 6)];
    }
}

// Write stage registers into LDS buffer `buf`; returns whether any lo unit of
// this thread is non-zero.
__device__ __forceinline__ bool stage_store(const StageRegs& R, uint8_t* buf) {
    const int t = threadIdx.x;
    uint4* A = reinterpret_cast<uint4*>(buf);
    A[t] = R.a0;
    A[t + 256] = R.a1;
    if (t < 128) {
        uint4* B = reinterpret_cast<uint4*>(buf + kGemmStageA + kGemmStageSeeds) + t * 4;
        const uint32_t w[4] = {R.q.x, R.q.y, R.q.z, R.q.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) B[d] = __builtin_bit_cast(uint4, q4_word_to_bf16x8(w[d]));
    } else {
        const int i = t - 128;
        reinterpret_cast<float*>(buf + kGemmStageA)[i] = R.seed;
        reinterpret_cast<float*>(buf + kGemmStageA + kGemmStageSeeds + kGemmStageB)[i] = f16_bits_to_f32(R.sc);
    }
    const uint4 lo = R.a1;  // units t + 256 are all lo parts
    return (lo.x | lo.y | lo.z | lo.w) != 0u;
}

template <int MODE, int RS>
__device__ __forceinline__ void gemm_body(const GemmArgs& a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const LayerView& L = a.L;
    const int H = L.hidden, I = L.inter, k = L.top_k;
    const int ti = blockIdx.x / a.nblocks, nb = blockIdx.x - ti * a.nblocks;
    const int count = dptr<const int>(a.W.meta)[2];
    if (ti >= count) return;
    const int tv = dptr<const int>(a.tiles)[ti];
    const ExpertEntry x = load_entry(a.W.et, tv >> 16);
    const int m0 = (tv & 0xffff) * kGemmBM;
    const int mvalid = min(kGemmBM, x.ntok - m0);
    const int K = MODE == 0 ? H : I;         // reduction width
    const int NR = MODE == 0 ? I : H;        // rows of each matrix
    const int n0 = nb * (MODE == 0 ? kGemmRows / 2 : kGemmRows);
    const int ng = K >> 5, ngp = frag_ngp(K);
    const uint64_t ib = (uint64_t)image_bytes(K);
    const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    float* out = dptr<float>(a.out);
    if (x.blob == 0) {  // a routed expert without a slot: flag it, contribute zeros
        if (tid == 0 && nb == 0) atomicOr(dptr<int>(a.W.meta) + 1, kErrMissingExpert);
        const int rows = MODE == 0 ? kGemmRows / 2 : kGemmRows;
        for (int e = tid; e < mvalid * rows; e += blockDim.x) {
            const int m = e / rows, r = n0 + e - m * rows;
            if (r < NR) out[(size_t)(x.p0 + m0 + m) * NR + r] = 0.0f;
        }
        return;
    }
    uint64_t* rowimg = reinterpret_cast<uint64_t*>(lds + 2 * kGemmStage);
    if (tid < kGemmBM) {
        const int m = min(tid, mvalid - 1);  // rows past the block repeat its last token
        const int pos = x.p0 + m0 + m;
        rowimg[tid] = MODE == 0 ? a.a_img + (uint64_t)(dptr<const int>(a.W.perm)[pos] / k) * ib
                                : a.a_img + (uint64_t)pos * ib;
    }
    const Region r0 = region_at(x.blob + (MODE == 0 ? L.gate_off : L.down_off), NR, K, RS);
    const Region r1 = region_at(x.blob + (MODE == 0 ? L.up_off : L.down_off), NR, K, RS);
    __syncthreads();

    float acc[8][4];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t][0] = acc[t][1] = acc[t][2] = acc[t][3] = 0.0f;

    StageRegs R;
    stage_load<MODE, RS>(R, rowimg, r0, r1, n0, ngp, 0);
    bool lo_any = __syncthreads_or(stage_store(R, lds));
    for (int g = 0; g < ng; ++g) {
        uint8_t* cur = lds + (g & 1) * kGemmStage;
        // the next stage's loads go out first (the last stage is loaded twice)
        stage_load<MODE, RS>(R, rowimg, r0, r1, n0, ngp, min(g + 1, ng - 1));
        {
            const uint4* A = reinterpret_cast<const uint4*>(cur);
            const int am = 16 * wave + (lane & 15), kb = lane >> 4;
            const uint4 ahi = A[(0 * kGemmBM + am) * 4 + kb];
            const uint4 alo = A[(1 * kGemmBM + am) * 4 + kb];
            const float* sd = reinterpret_cast<const float*>(cur + kGemmStageA);
            const int cm = 16 * wave + 4 * kb;  // the lane's C rows cm .. cm+3
            const float4 sh = *reinterpret_cast<const float4*>(sd + cm);
            const float4 sl = *reinterpret_cast<const float4*>(sd + kGemmBM + cm);
            const uint4* B = reinterpret_cast<const uint4*>(cur + kGemmStageA + kGemmStageSeeds);
            const float* S = reinterpret_cast<const float*>(cur + kGemmStageA + kGemmStageSeeds + kGemmStageB);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int row = 16 * t + (lane & 15);
                const bf16x8_t b = __builtin_bit_cast(bf16x8_t, B[row * 4 + kb]);
                f32x4_t c;
                c[0] = sh.x + sl.x;
                c[1] = sh.y + sl.y;
                c[2] = sh.z + sl.z;
                c[3] = sh.w + sl.w;
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ahi), b, c, 0, 0, 0);
                if (lo_any) c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, alo), b, c, 0, 0, 0);
                const float s = S[row];
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][i] = __builtin_fmaf(s, c[i], acc[t][i]);
            }
        }
        // the other buffer was last read in the previous iteration, which every
        // wave finished before that iteration's closing barrier
        lo_any = __syncthreads_or(stage_store(R, lds + ((g + 1) & 1) * kGemmStage));
    }

    // epilogue: lane holds C rows cm + i (tokens) of column lane & 15 in every row tile
    const int cm = 16 * wave + 4 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = cm + i;
        if (m >= mvalid) continue;
        float* orow = out + (size_t)(x.p0 + m0 + m) * NR;
        if (MODE == 0) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int r = n0 + 16 * t + (lane & 15);
                const float gg = acc[t][i], uu = acc[t + 4][i];
                if (r < NR) orow[r] = gg / (1.0f + expf(-gg)) * uu;
            }
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int r = n0 + 16 * t + (lane & 15);
                if (r < NR) orow[r] = acc[t][i];
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

// act rows (dispatch order) into fragment images for the down GEMM: 8 rows
// per workgroup, 32 sub-groups per row at a time.
extern "C" __global__ void __launch_bounds__(256) lp_gemm_actimg(const GemmArgs a) {
    const int I = a.L.inter;
    const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int total = a.T * a.L.top_k;
    if (row >= total) return;
    const float* src = dptr<const float>(a.W.act) + (size_t)row * I;
    uint8_t* img = dptr<uint8_t>(a.W.actimg) + (size_t)row * image_bytes(I);
    for (int g = threadIdx.x & 31; g < frag_ngp(I); g += 32) write_image_group(src, I, g, img);
}

extern "C" __global__ void __launch_bounds__(256) lp_gemm_gateup(const GemmArgs a) {
#define LP_G(rs) gemm_body<0, rs>(a)
    LP_BY_RS(a.L.group, LP_G)
#undef LP_G
}

extern "C" __global__ void __launch_bounds__(256) lp_gemm_down(const GemmArgs a) {
#define LP_G(rs) gemm_body<1, rs>(a)
    LP_BY_RS(a.L.group, LP_G)
#undef LP_G
}
