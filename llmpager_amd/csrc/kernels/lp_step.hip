// gfx950 kernels of the fused decode step around the MoE layer: the
// reference's Decoder::step (crates/llmpager-run/src/decode.rs:275-301)
// issues rmsnorm, three bf16_gemv, two per-head rmsnorm, two rope, kv_append,
// attn_decode, bf16_gemv, add and rmsnorm per layer, each a launch of its own
// (decode.cu:17-339).  Here the same arithmetic is these launches:
//
//   lp_rmsnorm_gemv      y_i = W_i . rmsnorm(x, ln) for up to three bf16
//                        matrices sharing the input (q / k / v; the lm_head)
//   lp_attn_fused        per-head q / k RMSNorm and NeoX RoPE, the token's k / v
//                        appended to the fp16 caches, GQA decode attention
//   lp_gemv_add_rmsnorm  h += W . a, then hn = rmsnorm(h, ln) (the o
//                        projection, the residual add and the next norm)
//   lp_attn_block        the last two in one launch (two per attention block
//                        with lp_rmsnorm_gemv)
//
// Work is handed between workgroups of one launch the way the fused routing
// kernel does it: agent-scope stores, a relaxed arrival counter in the
// stream's counter slot that the last arrival resets, then loads that see
// the stores (agent-scope loads, or plain loads of data that nothing on the
// reading XCD has read since the launch began).
#include "lp_device.h"

using namespace lp;
using namespace lpk;

namespace {

// One arrival at *cnt per workgroup (every thread calls it); returns the
// workgroup's arrival order, n - 1 for the last, which resets the counter.
// Each wave first waits until its own stores have completed.
__device__ __forceinline__ int arrival_order(int* cnt, int n, int* flag) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const int o = atomicAdd(cnt, 1);
        if (o == n - 1) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = o;
    }
    __syncthreads();
    return *flag;
}

__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o >= 1; o >>= 1) v += shfl_xor(v, o);
    return v;
}

// sum over the workgroup (red: 4 floats of LDS); ends with a barrier
__device__ __forceinline__ float block_sum4(float v, float* red) {
    v = wave_sum(v);
    if (lane_id() == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float t = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
    return t;
}

__device__ __forceinline__ uint16_t f16_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// ---------------------------------------------------------------------------
// bf16 GEMV rows.  Lane l holds the input's 8-column chunks l, l + 64, ...
// (CPL of them, zero past cols) and loads the same chunks of each row as one
// 16-byte piece: each load instruction of a wave reads 1 KB of the row.  The
// dot product is the fused multiply-add chain of lp_bf16_gemv (chunk by chunk,
// column order inside a chunk), then a butterfly over the 64 lanes.
// ---------------------------------------------------------------------------
template <int CPL>
__device__ __forceinline__ void load_vec(uint64_t x, int cols, float (&v)[CPL][8]) {
    const int lane = lane_id();
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = 8 * (lane + 64 * j);
        float4 lo = {0.0f, 0.0f, 0.0f, 0.0f}, hi = lo;
        if (c < cols) {
            lo = gptr<float4>(x)[c >> 2];
            hi = gptr<float4>(x)[(c >> 2) + 1];
        }
        v[j][0] = lo.x, v[j][1] = lo.y, v[j][2] = lo.z, v[j][3] = lo.w;
        v[j][4] = hi.x, v[j][5] = hi.y, v[j][6] = hi.z, v[j][7] = hi.w;
    }
}

template <int CPL>
__device__ __forceinline__ void load_row(uint64_t row, int cols, bool ok, uint4 (&w)[CPL]) {
    const int lane = lane_id();
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c8 = lane + 64 * j;
        w[j] = make_uint4(0, 0, 0, 0);
        if (ok && 8 * c8 < cols) w[j] = gptr<uint4>(row)[c8];
    }
}

template <int CPL>
__device__ __forceinline__ float row_dot(const uint4 (&w)[CPL], const float (&x)[CPL][8]) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const uint32_t u[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc = __builtin_fmaf(bf16_to_f32(u[i] & 0xffffu), x[j][2 * i], acc);
            acc = __builtin_fmaf(bf16_to_f32(u[i] >> 16), x[j][2 * i + 1], acc);
        }
    }
    return wave_sum(acc);
}

constexpr int kGemvRowsPerWave = kFusedGemvRowsPerWave;

// rows [seg0 | seg1 | seg2] of RmsNormGemvArgs: the matrix, output and local
// row of global row r (uniform across the wave)
struct RowRef {
    uint64_t w, y;
    int row;
    bool ok;
};

__device__ __forceinline__ RowRef row_ref(const RmsNormGemvArgs& a, int r) {
    RowRef o{0, 0, 0, false};
    if (r < a.rows0) {
        o = RowRef{a.w0, a.y0, r, true};
    } else if (r < a.rows0 + a.rows1) {
        o = RowRef{a.w1, a.y1, r - a.rows0, true};
    } else if (r < a.rows0 + a.rows1 + a.rows2) {
        o = RowRef{a.w2, a.y2, r - a.rows0 - a.rows1, true};
    }
    return o;
}

template <int CPL>
__device__ __forceinline__ void rmsnorm_gemv_body(const RmsNormGemvArgs& a) {
    const int wave = threadIdx.x >> 6, lane = lane_id();
    const int r0 = (blockIdx.x * 4 + wave) * kGemvRowsPerWave;
    // the input first (it is in L2), then the rows' loads stay in flight
    // while the norm is taken
    float x[CPL][8];
    load_vec<CPL>(a.x, a.cols, x);
    float g[CPL][8];
    if (a.ln) load_vec<CPL>(a.ln, a.cols, g);
    RowRef rr[kGemvRowsPerWave];
    uint4 w[kGemvRowsPerWave][CPL];
#pragma unroll
    for (int r = 0; r < kGemvRowsPerWave; ++r) {
        rr[r] = row_ref(a, r0 + r);
        load_row<CPL>(rr[r].w + (uint64_t)rr[r].row * a.cols * 2, a.cols, rr[r].ok, w[r]);
    }
    if (a.ln) {
        // RMSNorm (decode.cu:17-41): x * (1 / sqrt(mean(x^2) + eps)) * g;
        // every wave holds the whole input, so each takes the sum itself
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(x[j][i], x[j][i], ss);
        const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)a.cols + a.eps);
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) x[j][i] = x[j][i] * inv * g[j][i];
    }
#pragma unroll
    for (int r = 0; r < kGemvRowsPerWave; ++r) {
        const float y = row_dot<CPL>(w[r], x);
        if (lane == 0 && rr[r].ok) gptr_w<float>(rr[r].y)[rr[r].row] = y;
    }
}

template <int CPL>
__device__ __forceinline__ void gemv_add_rmsnorm_body(const GemvAddRmsNormArgs& a) {
    __shared__ float red[4];
    __shared__ int flag;
    const int wave = threadIdx.x >> 6, lane = lane_id();
    const int r0 = (blockIdx.x * 4 + wave) * kGemvRowsPerWave;
    float x[CPL][8];
    load_vec<CPL>(a.x, a.cols, x);
    uint4 w[kGemvRowsPerWave][CPL];
#pragma unroll
    for (int r = 0; r < kGemvRowsPerWave; ++r)
        load_row<CPL>(a.w + (uint64_t)(r0 + r) * a.cols * 2, a.cols, r0 + r < a.rows, w[r]);
    float* h = reinterpret_cast<float*>(a.h);
#pragma unroll
    for (int r = 0; r < kGemvRowsPerWave; ++r) {
        const float y = row_dot<CPL>(w[r], x);
        // the residual add (decode.cu:44-53 with s = 1: a[i] + b[i])
        if (lane == 0 && r0 + r < a.rows) agent_store(h + r0 + r, h[r0 + r] + y);
    }
    int* cnt = reinterpret_cast<int*>(a.sync) + kStepSyncGemv;
    if (arrival_order(cnt, gridDim.x, &flag) != (int)gridDim.x - 1) return;
    // the last workgroup: hn = rmsnorm(h, ln) over the whole row, every
    // load issued before the first is used
    constexpr int kPer = kFusedGemvMaxRows / 256;
    const float* ln = reinterpret_cast<const float*>(a.ln);
    float hv[kPer], gv[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = threadIdx.x + 256 * k;
        hv[k] = i < a.rows ? agent_load(h + i) : 0.0f;
        gv[k] = i < a.rows ? ln[i] : 0.0f;
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; ++k) ss = __builtin_fmaf(hv[k], hv[k], ss);
    const float inv = 1.0f / sqrtf(block_sum4(ss, red) / (float)a.rows + a.eps);
    float* hn = reinterpret_cast<float*>(a.hn);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = threadIdx.x + 256 * k;
        if (i < a.rows) hn[i] = hv[k] * inv * gv[k];
    }
}

}  // namespace

#define LP_GEMV_KERNELS(CPL)                                                                               \
    extern "C" __global__ void __launch_bounds__(256) lp_rmsnorm_gemv_c##CPL(const RmsNormGemvArgs a) {    \
        rmsnorm_gemv_body<CPL>(a);                                                                         \
    }                                                                                                      \
    extern "C" __global__ void __launch_bounds__(256) lp_gemv_add_rmsnorm_c##CPL(const GemvAddRmsNormArgs a) { \
        gemv_add_rmsnorm_body<CPL>(a);                                                                     \
    }
LP_GEMV_KERNELS(1)
LP_GEMV_KERNELS(2)
LP_GEMV_KERNELS(4)
LP_GEMV_KERNELS(8)
#undef LP_GEMV_KERNELS

// ---------------------------------------------------------------------------
// Fused GQA decode attention for head_dim 128 and G query heads per KV head
// (the reference's rmsnorm per head, rope, kv_append and attn_decode_f16kv,
// decode.rs:283-294).  Grid (splits, kv_heads), 4 waves.  Workgroup (s, g):
//
//   prologue  the G query heads of KV head g: RMSNorm with q_norm, NeoX RoPE
//             at pos (decode.cu:17-41, 145-167), into LDS; the split holding
//             pos also takes k's head g (k_norm, RoPE) and v's, rounds both
//             to fp16 and writes them into the caches at row pos (decode.cu:
//             242-261).  The first chunk's cache loads are issued first, the
//             rotation angles are computed while the loads are in flight.
//   chunks    of 64 positions, 16 per wave.  Scores on MFMA
//             (v_mfma_f32_16x16x32_f16): A = the query heads (M, padded to
//             16), the fp32 values split into fp16 hi + lo (two MFMAs per
//             step, 22 significant bits), B = 16 cache rows (N), loaded as
//             16-byte row pieces; D lane (n, kb) value v is head 4 kb + v at
//             row n.  Online softmax per head over the wave's rows (DPP
//             reductions across each 16-lane row); the context on the VALU,
//             lane l owning dimensions 2 l and 2 l + 1 of all 16 rows, the
//             probabilities read from LDS.  Row pos comes from LDS, not from
//             the cache being written.
//   merge     the four waves' states in LDS; one split writes the output, more
//             write partial records {max, sum, acc[128]} to the scratch and
//             the last of them to arrive (a counter per KV head) merges them,
//             its record loads issued in one burst.
// ---------------------------------------------------------------------------
namespace {

constexpr int kHd = 128;

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4_t mfma_f16(const uint4& a, const uint4& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
}

__device__ __forceinline__ uint32_t pack16(uint16_t lo, uint16_t hi) { return (uint32_t)lo | ((uint32_t)hi << 16); }

// a value of another lane of the same 16-lane row, through DPP: quad_perm
// [1,0,3,2] (lane ^ 1), [2,3,0,1] (lane ^ 2), row_ror:4, row_ror:8
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// the sum / maximum over each row of 16 lanes, in every lane of the row
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp<0xb1>(v);
    v += dpp<0x4e>(v);
    v += dpp<0x124>(v);
    return v + dpp<0x128>(v);
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp<0xb1>(v));
    v = fmaxf(v, dpp<0x4e>(v));
    v = fmaxf(v, dpp<0x124>(v));
    return fmaxf(v, dpp<0x128>(v));
}

// The attention output leaves by agent-scope stores when another workgroup
// of the launch reads it (done != null); the workgroup that completes a KV
// head's output then adds one to *done.
template <int G>
__device__ __forceinline__ void attn_fused_body(const AttnFusedArgs& a, int sp, int g, int* done) {
    constexpr int STEPS = kHd / 32;
    __shared__ __align__(16) float qf[G][kHd];
    __shared__ __align__(16) uint4 qb[2][STEPS][64];
    __shared__ __align__(16) uint16_t kvn[2][kHd];
    __shared__ __align__(16) float pl[4][16][16];  // wave, head, row
    __shared__ float al[4][16];                     // wave, head: this chunk's rescale
    __shared__ __align__(16) float wacc[4][G][kHd];
    __shared__ float wm[4][16], wl[4][16];
    __shared__ float mw[16 * kAttnFusedMaxSplits];
    __shared__ int flag;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const int n = lane & 15, kb = lane >> 4;
    const int pos = a.pos, seq = pos + 1;
    const int nch = (seq + 63) >> 6;
    const int c0 = sp * a.cps, c1 = min(nch, c0 + a.cps);
    const bool owner = c1 == nch;  // the last split holds position pos
    const uint64_t kc = a.kcache + (uint64_t)g * a.max_seq * kHd * 2;
    const uint64_t vc = a.vcache + (uint64_t)g * a.max_seq * kHd * 2;
    // the valid rows of head g's caches through raw buffers: rows past pos
    // read zero
    const int nbytes = __builtin_amdgcn_readfirstlane(seq * kHd * 2);
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(uniform_u64(kc)), (short)0, nbytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(uniform_u64(vc)), (short)0, nbytes, kBufferWord3);
    uint4 B[STEPS];
    uint32_t V[16];  // dimensions 2 lane, 2 lane + 1 of the wave's 16 rows
    auto load_k = [&](int c) {
        const uint32_t off = (uint32_t)(64 * c + 16 * wave + n) * (kHd * 2) + 16u * (uint32_t)kb;
#pragma unroll
        for (int j = 0; j < STEPS; ++j)
            B[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, (int)(off + 64u * j), 0, 0));
    };
    auto load_v = [&](int c) {
        const uint32_t off = (uint32_t)(64 * c + 16 * wave) * (kHd * 2) + 4u * (uint32_t)lane;
#pragma unroll
        for (int r = 0; r < 16; ++r) V[r] = __builtin_amdgcn_raw_buffer_load_b32(rv, (int)(off + (kHd * 2) * r), 0, 0);
    };

    // ---- prologue: the raw projections (written by the previous launch)
    const int nvec = G + (owner ? 1 : 0);
    constexpr int kPasses = (G + 1 + 7) / 8;
    const int j = tid & 31;
    float xr[kPasses][4];
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        const int vi = 8 * p + (tid >> 5);
        const float* src = vi < G ? reinterpret_cast<const float*>(a.q) + ((size_t)g * G + vi) * kHd
                                  : reinterpret_cast<const float*>(a.k) + (size_t)g * kHd;
#pragma unroll
        for (int u = 0; u < 4; ++u) xr[p][u] = vi < nvec ? src[j + 32 * u] : 0.0f;
    }
    float vr = 0.0f;
    if (owner && tid < kHd) vr = reinterpret_cast<const float*>(a.v)[(size_t)g * kHd + tid];
    float gq[4] = {1.0f, 1.0f, 1.0f, 1.0f}, gk[4] = {1.0f, 1.0f, 1.0f, 1.0f};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        if (a.q_norm) gq[u] = reinterpret_cast<const float*>(a.q_norm)[j + 32 * u];
        if (a.k_norm) gk[u] = reinterpret_cast<const float*>(a.k_norm)[j + 32 * u];
    }
    load_k(c0);
    load_v(c0);
    // NeoX rotate-half: pairs (i, i + 64) for i = j, j + 32
    float cs[2], sn[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int i = j + 32 * u;
        const float freq = powf(a.rope_base, -2.0f * (float)i / (float)kHd);
        const float ang = (float)pos * freq;
        cs[u] = cosf(ang);
        sn[u] = sinf(ang);
    }
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        const int vi = 8 * p + (tid >> 5);
        const bool isk = vi == G;
        float x[4] = {xr[p][0], xr[p][1], xr[p][2], xr[p][3]};
        if (isk ? a.k_norm != 0 : a.q_norm != 0) {
            float ss = 0.0f;
#pragma unroll
            for (int u = 0; u < 4; ++u) ss = __builtin_fmaf(x[u], x[u], ss);
            ss = row16_sum(ss);
            ss += shfl_xor(ss, 16);
            const float inv = 1.0f / sqrtf(ss / (float)kHd + a.eps);
#pragma unroll
            for (int u = 0; u < 4; ++u) x[u] = x[u] * inv * (isk ? gk[u] : gq[u]);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const float x1 = x[u], x2 = x[u + 2];
            x[u] = x1 * cs[u] - x2 * sn[u];
            x[u + 2] = x1 * sn[u] + x2 * cs[u];
        }
        if (vi < G) {
#pragma unroll
            for (int u = 0; u < 4; ++u) qf[vi][j + 32 * u] = x[u];
        } else if (isk && owner) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint16_t hb = f16_bits(x[u]);
                kvn[0][j + 32 * u] = hb;
                gptr_w<uint16_t>(kc)[(size_t)pos * kHd + j + 32 * u] = hb;
            }
        }
    }
    if (owner && tid < kHd) {
        const uint16_t hb = f16_bits(vr);
        kvn[1][tid] = hb;
        gptr_w<uint16_t>(vc)[(size_t)pos * kHd + tid] = hb;
    }
    __syncthreads();
    // A fragments: step j, lane (m, kb) holds q[m][32 j + 8 kb .. + 7] as
    // fp16 hi and lo; heads past G are zero
    {
        const int st = tid >> 6, m = lane & 15, k8 = lane >> 4;
        uint16_t hi[8], lo[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float v = m < G ? qf[m < G ? m : 0][32 * st + 8 * k8 + i] : 0.0f;
            hi[i] = f16_bits(v);
            lo[i] = f16_bits(v - f16_bits_to_f32(hi[i]));
        }
        qb[0][st][lane] = make_uint4(pack16(hi[0], hi[1]), pack16(hi[2], hi[3]), pack16(hi[4], hi[5]),
                                     pack16(hi[6], hi[7]));
        qb[1][st][lane] = make_uint4(pack16(lo[0], lo[1]), pack16(lo[2], lo[3]), pack16(lo[4], lo[5]),
                                     pack16(lo[6], lo[7]));
    }
    __syncthreads();
    uint4 ah[STEPS], alo[STEPS];
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
        ah[st] = qb[0][st][lane];
        alo[st] = qb[1][st][lane];
    }

    // ---- chunks
    float m_run[4], l_run[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) m_run[v] = -INFINITY, l_run[v] = 0.0f;
    float acc[G][2];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) acc[hh][0] = acc[hh][1] = 0.0f;
    for (int c = c0; c < c1; ++c) {
        const int rowk = 64 * c + 16 * wave + n;
        if (rowk == pos) {
#pragma unroll
            for (int st = 0; st < STEPS; ++st) B[st] = *reinterpret_cast<const uint4*>(&kvn[0][32 * st + 8 * kb]);
        }
        f32x4_t s4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            s4 = mfma_f16(ah[st], B[st], s4);
            s4 = mfma_f16(alo[st], B[st], s4);
        }
        if (c + 1 < c1) load_k(c + 1);
        // online softmax: lane (n, kb) value v is head 4 kb + v at row n
        const bool valid = rowk < seq;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float sv = valid ? s4[v] * a.scale : -INFINITY;
            const float mn = fmaxf(m_run[v], row16_max(sv));
            const bool none = mn == -INFINITY;
            const float alpha = none ? 1.0f : exp_hw(m_run[v] - mn);
            const float p = none ? 0.0f : exp_hw(sv - mn);
            l_run[v] = __builtin_fmaf(l_run[v], alpha, row16_sum(p));
            m_run[v] = mn;
            pl[wave][4 * kb + v][n] = p;
            if (n == 0) al[wave][4 * kb + v] = alpha;
        }
        __builtin_amdgcn_wave_barrier();
        // context: dimensions 2 lane, 2 lane + 1 of the wave's 16 rows
        const int r_pos = pos - (64 * c + 16 * wave);  // the new row's index here, if any
        if (r_pos >= 0 && r_pos < 16) {
            const uint32_t nv = *reinterpret_cast<const uint32_t*>(&kvn[1][2 * lane]);
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (r == r_pos) V[r] = nv;
        }
        float vf[16][2];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            vf[r][0] = f16_bits_to_f32(V[r] & 0xffffu);
            vf[r][1] = f16_bits_to_f32(V[r] >> 16);
        }
        if (c + 1 < c1) load_v(c + 1);
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            const float sc = al[wave][hh];
            float t0 = acc[hh][0] * sc, t1 = acc[hh][1] * sc;
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float4 p4 = *reinterpret_cast<const float4*>(&pl[wave][hh][4 * q4]);
                const float pv[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    t0 = __builtin_fmaf(pv[i], vf[4 * q4 + i][0], t0);
                    t1 = __builtin_fmaf(pv[i], vf[4 * q4 + i][1], t1);
                }
            }
            acc[hh][0] = t0, acc[hh][1] = t1;
        }
        __builtin_amdgcn_wave_barrier();
    }
    // ---- the wave's state to LDS
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
        *reinterpret_cast<float2*>(&wacc[wave][hh][2 * lane]) = make_float2(acc[hh][0], acc[hh][1]);
    if (n == 0) {
#pragma unroll
        for (int v = 0; v < 4; ++v) wm[wave][4 * kb + v] = m_run[v], wl[wave][4 * kb + v] = l_run[v];
    }
    __syncthreads();
    float* out = reinterpret_cast<float*>(a.out);
    float* scr = reinterpret_cast<float*>(a.scratch);
    constexpr int kRec = kAttnFusedRec;
    for (int o = tid; o < G * kHd; o += 256) {
        const int hh = o / kHd, d = o % kHd;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, wm[w][hh]);
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float e = exp_hw(wm[w][hh] - M);  // a wave with no valid row: e^-inf = 0
            L = __builtin_fmaf(e, wl[w][hh], L);
            A = __builtin_fmaf(e, wacc[w][hh][d], A);
        }
        const size_t head = (size_t)g * G + hh;
        if (a.splits == 1) {
            if (done)
                agent_store(out + head * kHd + d, A / L);
            else
                out[head * kHd + d] = A / L;
        } else {
            float* rec = scr + head * a.scratch_stride + (size_t)sp * kRec;
            agent_store(rec + d, A);
            if (d == 0) {
                agent_store(rec + kHd, M);
                agent_store(rec + kHd + 1, L);
            }
        }
    }
    if (a.splits == 1) {
        if (done) signal_count(done);
        return;
    }
    int* cnt = reinterpret_cast<int*>(a.sync) + kStepSyncAttn + kSyncStride * g;
    if (arrival_order(cnt, a.splits, &flag) != a.splits - 1) return;
    // ---- the last split of head group g merges the records.  They were
    // written in this launch with agent-scope stores and nothing on this XCD
    // has read them since the launch began, so plain loads see them.  Every
    // load is issued at once: the {max, sum} pairs (32 lanes per head, lane s
    // holding split s) and each thread's accumulators (4 dimensions of one
    // head: 16-byte loads) of up to 16 splits; the weights e^(m_s - M) /
    // sum_s e^(m_s - M) l_s then go through LDS to the threads that need them.
    const int S = a.splits;
    constexpr int kOut = G * kHd / 4 / 256 > 0 ? G * kHd / 4 / 256 : 1;
    constexpr int kWP = (G + 7) / 8;
    float mr[kWP], lr[kWP];
#pragma unroll
    for (int p = 0; p < kWP; ++p) {
        const int hh = 8 * p + (tid >> 5), s = tid & 31;
        const bool on = hh < G && s < S;
        const float* rec = scr + ((size_t)g * G + (hh < G ? hh : 0)) * a.scratch_stride + (size_t)s * kRec + kHd;
        float2 ml = make_float2(-INFINITY, 0.0f);
        if (on) ml = *gptr<float2>(reinterpret_cast<uint64_t>(rec));
        mr[p] = ml.x;
        lr[p] = ml.y;
    }
    float4 num[kOut];
#pragma unroll
    for (int i = 0; i < kOut; ++i) num[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int s0 = 0; s0 < S; s0 += 16) {
        float4 v[16][kOut];
#pragma unroll
        for (int k = 0; k < 16; ++k)
#pragma unroll
            for (int i = 0; i < kOut; ++i) {
                const int o = tid + 256 * i, hh = o >> 5, d4 = o & 31;
                const float* rec = scr + ((size_t)g * G + (hh < G ? hh : 0)) * a.scratch_stride +
                                   (size_t)(s0 + k) * kRec + 4 * d4;
                v[k][i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (s0 + k < S && hh < G) v[k][i] = *gptr<float4>(reinterpret_cast<uint64_t>(rec));
            }
        if (s0 == 0) {
#pragma unroll
            for (int p = 0; p < kWP; ++p) {
                const int hh = 8 * p + (tid >> 5), s = tid & 31;
                float M = row16_max(mr[p]);
                M = fmaxf(M, shfl_xor(M, 16));
                const float e = s < S ? exp_hw(mr[p] - M) : 0.0f;
                float den = row16_sum(e * lr[p]);
                den += shfl_xor(den, 16);
                if (hh < G && s < S) mw[hh * kAttnFusedMaxSplits + s] = e / den;
            }
            __syncthreads();
        }
#pragma unroll
        for (int k = 0; k < 16; ++k)
#pragma unroll
            for (int i = 0; i < kOut; ++i) {
                const int hh = (tid + 256 * i) >> 5;
                if (s0 + k < S && hh < G) {
                    const float wt = mw[hh * kAttnFusedMaxSplits + s0 + k];
                    num[i].x = __builtin_fmaf(wt, v[k][i].x, num[i].x);
                    num[i].y = __builtin_fmaf(wt, v[k][i].y, num[i].y);
                    num[i].z = __builtin_fmaf(wt, v[k][i].z, num[i].z);
                    num[i].w = __builtin_fmaf(wt, v[k][i].w, num[i].w);
                }
            }
    }
#pragma unroll
    for (int i = 0; i < kOut; ++i) {
        const int o = tid + 256 * i, hh = o >> 5, d4 = o & 31;
        if (hh < G) {
            float* po = out + ((size_t)g * G + hh) * kHd + 4 * d4;
            if (done) {
                agent_store(po, num[i].x);
                agent_store(po + 1, num[i].y);
                agent_store(po + 2, num[i].z);
                agent_store(po + 3, num[i].w);
            } else {
                *reinterpret_cast<float4*>(po) = num[i];
            }
        }
    }
    if (done) signal_count(done);
}

}  // namespace

#define LP_ATTN_FUSED(G)                                                                             \
    extern "C" __global__ void __launch_bounds__(256) lp_attn_fused_g##G(const AttnFusedArgs a) {  \
        attn_fused_body<G>(a, blockIdx.x, blockIdx.y, nullptr);                                      \
    }
LP_ATTN_FUSED(1)
LP_ATTN_FUSED(2)
LP_ATTN_FUSED(4)
LP_ATTN_FUSED(8)
LP_ATTN_FUSED(16)
#undef LP_ATTN_FUSED

// ---------------------------------------------------------------------------
// The attention block's tail in one launch: lp_attn_fused on workgroups
// [0, n_attn) (split s of KV head g at s + splits g), then the o projection,
// the residual add and the post-attention norm (lp_gemv_add_rmsnorm) on the
// workgroups after them.  Those start by loading their rows of W_o, which do
// not depend on the attention, then wait for the attention's KV heads to be
// complete (a counter) and read its output with agent-scope loads.  The last
// of them resets the counter.
// ---------------------------------------------------------------------------
namespace {

constexpr int kBlockCpl = kFusedGemvMaxCols / 512;

template <int G>
__device__ __forceinline__ void attn_block_body(const AttnBlockArgs& b) {
    const AttnFusedArgs& a = b.at;
    int* sync = reinterpret_cast<int*>(a.sync);
    if ((int)blockIdx.x < b.n_attn) {
        attn_fused_body<G>(a, blockIdx.x % a.splits, blockIdx.x / a.splits, sync + kStepSyncDone);
        return;
    }
    __shared__ float red[4];
    __shared__ int flag;
    constexpr int CPL = kBlockCpl;
    const int wave = threadIdx.x >> 6, lane = lane_id();
    const int r0 = ((blockIdx.x - b.n_attn) * 4 + wave) * kBlockRowsPerWave;
    uint4 w[kBlockRowsPerWave][CPL];
#pragma unroll
    for (int r = 0; r < kBlockRowsPerWave; ++r)
        load_row<CPL>(b.wo + (uint64_t)(r0 + r) * b.cols * 2, b.cols, r0 + r < b.rows, w[r]);
    float hr[kBlockRowsPerWave];
#pragma unroll
    for (int r = 0; r < kBlockRowsPerWave; ++r) hr[r] = r0 + r < b.rows ? reinterpret_cast<const float*>(b.h)[r0 + r] : 0.0f;
    wait_count(sync + kStepSyncDone, a.kv_heads, sync + kStepSyncErr, b.spin_max);
    // the attention output: written in this launch with agent-scope stores,
    // and nothing on this XCD read it before they completed, so plain loads
    // see it
    float x[CPL][8];
    load_vec<CPL>(a.out, b.cols, x);
    float* h = reinterpret_cast<float*>(b.h);
#pragma unroll
    for (int r = 0; r < kBlockRowsPerWave; ++r) {
        const float y = row_dot<CPL>(w[r], x);
        if (lane == 0 && r0 + r < b.rows) agent_store(h + r0 + r, hr[r] + y);
    }
    const int n_o = (int)gridDim.x - b.n_attn;
    if (arrival_order(sync + kStepSyncGemv, n_o, &flag) != n_o - 1) return;
    // every workgroup has passed its wait: the counter starts the next launch at zero
    if (threadIdx.x == 0) agent_store(sync + kStepSyncDone, 0);
    constexpr int kPer = kFusedGemvMaxRows / 256;
    const float* ln = reinterpret_cast<const float*>(b.ln);
    float hv[kPer], gv[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = threadIdx.x + 256 * k;
        hv[k] = i < b.rows ? agent_load(h + i) : 0.0f;
        gv[k] = i < b.rows ? ln[i] : 0.0f;
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; ++k) ss = __builtin_fmaf(hv[k], hv[k], ss);
    const float inv = 1.0f / sqrtf(block_sum4(ss, red) / (float)b.rows + a.eps);
    float* hn = reinterpret_cast<float*>(b.hn);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = threadIdx.x + 256 * k;
        if (i < b.rows) hn[i] = hv[k] * inv * gv[k];
    }
}

}  // namespace

#define LP_ATTN_BLOCK(G)                                                                             \
    extern "C" __global__ void __launch_bounds__(256) lp_attn_block_g##G(const AttnBlockArgs a) {  \
        attn_block_body<G>(a);                                                                       \
    }
LP_ATTN_BLOCK(1)
LP_ATTN_BLOCK(2)
LP_ATTN_BLOCK(4)
LP_ATTN_BLOCK(8)
LP_ATTN_BLOCK(16)
#undef LP_ATTN_BLOCK
