// gfx950 kernels for the rest of the decode step around the MoE layer
// (crates/llmpager-cuda/kernels/decode.cu: RMSNorm, scale-add, KV append,
// NeoX RoPE, GQA decode attention over f32 or f16 caches, bf16 row gather)
// and for MLA absorbed decode (kernels/mla.cu: interleaved RoPE, attention
// over the shared latent cache, batched bf16 GEMV, strided copy), behind
// 1:1 launchers with the reference's argument meaning.  The arithmetic is
// this build's own: decode attention is split over positions (one workgroup
// per (head, split), partial records merged by a second kernel), and config
// 5's batched MLA decode over bf16 latent caches runs on MFMA.
#include "lp_device.h"

using namespace lp;
using namespace lpk;

namespace {

template <typename T>
__device__ __forceinline__ T* dptr(uint64_t a) {
    return reinterpret_cast<T*>(a);
}

// Sum / max over a workgroup of nw waves (red: nw floats of LDS).  Ends with a
// barrier, so LDS written before the call is visible after it.
__device__ __forceinline__ float block_sum(float v, float* red) {
    for (int o = 32; o >= 1; o >>= 1) v += shfl_xor(v, o);
    const int nw = (int)(blockDim.x >> 6);
    if (lane_id() == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
    for (int w = 0; w < nw; ++w) t += red[w];
    __syncthreads();
    return t;
}

__device__ __forceinline__ float block_max(float v, float* red) {
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, shfl_xor(v, o));
    const int nw = (int)(blockDim.x >> 6);
    if (lane_id() == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int w = 0; w < nw; ++w) t = fmaxf(t, red[w]);
    __syncthreads();
    return t;
}

__device__ __forceinline__ float half_bits_to_f32(uint32_t h) { return f16_bits_to_f32(h & 0xffffu); }

__device__ __forceinline__ uint16_t f32_to_half_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);  // round to nearest even
}

}  // namespace

// ---------------------------------------------------------------------------
// RMSNorm per row (decode.cu:17-41): y[r] = x[r] * 1/sqrt(mean(x[r]^2) + eps)
// * w.  One workgroup of 256 per row; w is shared by all rows; y may be x.
// ---------------------------------------------------------------------------
extern "C" __global__ void __launch_bounds__(256) lp_rmsnorm(const RmsNormArgs a) {
    __shared__ float red[4];
    const float* x = dptr<const float>(a.x) + (size_t)blockIdx.x * a.n;
    float* y = dptr<float>(a.y) + (size_t)blockIdx.x * a.n;
    const float* w = dptr<const float>(a.w);
    float acc = 0.0f;
    for (int i = threadIdx.x; i < a.n; i += 256) acc = __builtin_fmaf(x[i], x[i], acc);
    const float inv = 1.0f / sqrtf(block_sum(acc, red) / (float)a.n + a.eps);
    for (int i = threadIdx.x; i < a.n; i += 256) y[i] = x[i] * inv * w[i];
}

// a += s * b (decode.cu:44-53)
extern "C" __global__ void __launch_bounds__(256) lp_scale_add(const ScaleAddArgs a) {
    float* pa = dptr<float>(a.a);
    const float* pb = dptr<const float>(a.b);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += gridDim.x * blockDim.x)
        pa[i] = __builtin_fmaf(a.s, pb[i], pa[i]);
}

// The token's k / v ([kv_heads, head_dim]) into caches [kv_heads, max_seq,
// head_dim] at `pos` (decode.cu:57-77, 242-261); f16 caches round to
// nearest even.
extern "C" __global__ void __launch_bounds__(256) lp_kv_append_f32(const KvAppendArgs a) {
    const int total = a.kv_heads * a.head_dim;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int h = i / a.head_dim, d = i - h * a.head_dim;
        const size_t dst = ((size_t)h * a.max_seq + a.pos) * a.head_dim + d;
        dptr<float>(a.kcache)[dst] = dptr<const float>(a.k)[i];
        dptr<float>(a.vcache)[dst] = dptr<const float>(a.v)[i];
    }
}

extern "C" __global__ void __launch_bounds__(256) lp_kv_append_f16(const KvAppendArgs a) {
    const int total = a.kv_heads * a.head_dim;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int h = i / a.head_dim, d = i - h * a.head_dim;
        const size_t dst = ((size_t)h * a.max_seq + a.pos) * a.head_dim + d;
        dptr<uint16_t>(a.kcache)[dst] = f32_to_half_bits(dptr<const float>(a.k)[i]);
        dptr<uint16_t>(a.vcache)[dst] = f32_to_half_bits(dptr<const float>(a.v)[i]);
    }
}

// NeoX rotate-half RoPE in place over [heads, head_dim] (decode.cu:145-167):
// pair (i, i + hd/2) rotates by pos * base^(-2i/hd).  Library powf / cosf /
// sinf (the reference's fast-math intrinsics are approximations of these).
extern "C" __global__ void __launch_bounds__(256) lp_rope(const RopeArgs a) {
    const int half = a.head_dim >> 1;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < a.heads * half; idx += gridDim.x * blockDim.x) {
        const int h = idx / half, i = idx - h * half;
        const float freq = powf(a.base, -2.0f * (float)i / (float)a.head_dim);
        const float ang = (float)a.pos * freq;
        const float c = cosf(ang), s = sinf(ang);
        float* p = dptr<float>(a.x) + (size_t)h * a.head_dim;
        const float x1 = p[i], x2 = p[i + half];
        p[i] = x1 * c - x2 * s;
        p[i + half] = x1 * s + x2 * c;
    }
}

// out[n] = f32(table[row, :n]) (decode.cu:328-339)
extern "C" __global__ void __launch_bounds__(256) lp_bf16_row_to_f32(const RowArgs a) {
    const uint16_t* src = dptr<const uint16_t>(a.table) + (size_t)a.row * a.n;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += gridDim.x * blockDim.x)
        dptr<float>(a.out)[i] = bf16_to_f32(src[i]);
}

// Interleaved RoPE with a frequency table (mla.cu:22-45): pairs (2i, 2i+1) of
// the slice at `offset` in each of n_vecs vectors rotate by pos * inv_freq[i],
// both factors scaled by mscale.
extern "C" __global__ void __launch_bounds__(256) lp_mla_rope(const MlaRopeArgs a) {
    const float* fr = dptr<const float>(a.inv_freq);
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < a.n_vecs * a.half; idx += gridDim.x * blockDim.x) {
        const int v = idx / a.half, i = idx - v * a.half;
        const float ang = (float)a.pos * fr[i];
        const float c = cosf(ang) * a.mscale, s = sinf(ang) * a.mscale;
        float* p = dptr<float>(a.x) + (size_t)v * a.stride + a.offset + 2 * i;
        const float x1 = p[0], x2 = p[1];
        p[0] = x1 * c - x2 * s;
        p[1] = x1 * s + x2 * c;
    }
}

// Batched bf16 GEMV (mla.cu:120-148): y_b = W_b x_b, W_b = w + b w_stride
// [rows, cols] row-major, x_b = x + b x_stride, y_b = y + b y_stride (strides
// in elements).  One wave per row, lanes over 8-column chunks (16-byte loads
// when the row and x_b are 16-byte aligned), butterfly reduction.  Grid
// (ceil(rows / 4), batch).
extern "C" __global__ void __launch_bounds__(256) lp_bf16_gemv_batch(const Bf16GemvBatchArgs a) {
    const int b = blockIdx.y;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = lane_id();
    if (row >= a.rows) return;
    const uint16_t* w = dptr<const uint16_t>(a.w) + (size_t)b * a.w_stride + (size_t)row * a.cols;
    const float* x = dptr<const float>(a.x) + (size_t)b * a.x_stride;
    float acc = 0.0f;
    const bool vec = (a.cols & 7) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    if (vec) {
        for (int ch = lane; ch < (a.cols >> 3); ch += 64) {
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
    if (lane == 0) dptr<float>(a.y)[(size_t)b * a.y_stride + row] = acc;
}

// dst[v dst_stride + dst_off + i] = src[v src_stride + src_off + i]
// (mla.cu:153-166)
extern "C" __global__ void __launch_bounds__(256) lp_strided_copy(const StridedCopyArgs a) {
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < a.n_vecs * a.n; idx += gridDim.x * blockDim.x) {
        const int v = idx / a.n, i = idx - v * a.n;
        dptr<float>(a.dst)[(size_t)v * a.dst_stride + a.dst_off + i] =
            dptr<const float>(a.src)[(size_t)v * a.src_stride + a.src_off + i];
    }
}

// ---------------------------------------------------------------------------
// Decode attention, one query per head, split over positions (attn_decode_f32
// / _f16kv, decode.cu:172-325; mla_attn_decode_f32, mla.cu:51-111).  Grid
// (heads, splits), 256 threads.  Split s of head h takes positions
// [s span, min((s + 1) span, seq_len)): each thread scores whole positions
// (its key row against the query staged in LDS), the workgroup takes their
// max and the sum of exp(score - max), then each thread accumulates output
// dimensions over the split's positions.  One split writes out[h] = acc / sum;
// more write partial records {max, sum, acc[out_dim]} that lp_attn_combine
// merges (an empty split records {-inf, 0, 0...}).
// ---------------------------------------------------------------------------
namespace {

template <bool F16>
__device__ __forceinline__ float cache_at(uint64_t base, size_t i) {
    if constexpr (F16)
        return half_bits_to_f32(dptr<const uint16_t>(base)[i]);
    else
        return dptr<const float>(base)[i];
}

// dot(q, row) over n elements of an f32 or f16 cache row; vector loads when
// the row and n allow them
template <bool F16>
__device__ __forceinline__ float row_dot(const float* qs, uint64_t base, size_t row0, int n) {
    float dot = 0.0f;
    if constexpr (F16) {
        if ((n & 7) == 0 && ((base + row0 * 2) & 15) == 0) {
            const uint4* r = reinterpret_cast<const uint4*>(base + row0 * 2);
            for (int c = 0; c < (n >> 3); ++c) {
                const uint4 u = r[c];
                const uint32_t wv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    dot = __builtin_fmaf(qs[8 * c + 2 * j], half_bits_to_f32(wv[j]), dot);
                    dot = __builtin_fmaf(qs[8 * c + 2 * j + 1], half_bits_to_f32(wv[j] >> 16), dot);
                }
            }
            return dot;
        }
    } else {
        if ((n & 3) == 0 && ((base + row0 * 4) & 15) == 0) {
            const float4* r = reinterpret_cast<const float4*>(base + row0 * 4);
            for (int c = 0; c < (n >> 2); ++c) {
                const float4 u = r[c];
                dot = __builtin_fmaf(qs[4 * c], u.x, dot);
                dot = __builtin_fmaf(qs[4 * c + 1], u.y, dot);
                dot = __builtin_fmaf(qs[4 * c + 2], u.z, dot);
                dot = __builtin_fmaf(qs[4 * c + 3], u.w, dot);
            }
            return dot;
        }
    }
    for (int d = 0; d < n; ++d) dot = __builtin_fmaf(qs[d], cache_at<F16>(base, row0 + d), dot);
    return dot;
}

constexpr int kAttnMaxDot = 1024;

template <bool F16>
__device__ __forceinline__ void attn_split_body(const AttnArgs& a) {
    __shared__ float qs[kAttnMaxDot];
    __shared__ float sc[kAttnSpanMax];
    __shared__ float red[4];
    const int h = blockIdx.x, sp = blockIdx.y, tid = threadIdx.x;
    const uint64_t kv_off = (uint64_t)(h / a.group) * a.kv_stride;
    const float* q = dptr<const float>(a.q) + (size_t)h * a.dot_dim;
    for (int d = tid; d < a.dot_dim; d += 256) qs[d] = q[d];
    __syncthreads();
    const int p0 = sp * a.span;
    const int p1 = min(a.seq_len, p0 + a.span);
    float lmax = -INFINITY;
    for (int p = p0 + tid; p < p1; p += 256) {
        const float s = row_dot<F16>(qs, a.k, kv_off + (size_t)p * a.row_stride, a.dot_dim) * a.scale;
        sc[p - p0] = s;
        lmax = fmaxf(lmax, s);
    }
    const float m = block_max(lmax, red);
    float lsum = 0.0f;
    for (int p = p0 + tid; p < p1; p += 256) {
        const float e = expf(sc[p - p0] - m);
        sc[p - p0] = e;
        lsum += e;
    }
    const float l = block_sum(lsum, red);
    float* part = dptr<float>(a.scratch) + (size_t)h * a.scratch_stride + (size_t)sp * (a.out_dim + 2);
    for (int d = tid; d < a.out_dim; d += 256) {
        float acc = 0.0f;
        for (int p = p0; p < p1; ++p)
            acc = __builtin_fmaf(sc[p - p0], cache_at<F16>(a.v, kv_off + (size_t)p * a.row_stride + d), acc);
        if (a.splits == 1)
            dptr<float>(a.out)[(size_t)h * a.out_dim + d] = acc * (1.0f / l);
        else
            part[2 + d] = acc;
    }
    if (a.splits > 1 && tid == 0) {
        part[0] = m;
        part[1] = l;
    }
}

}  // namespace

extern "C" __global__ void __launch_bounds__(256) lp_attn_split_f32(const AttnArgs a) { attn_split_body<false>(a); }
extern "C" __global__ void __launch_bounds__(256) lp_attn_split_f16(const AttnArgs a) { attn_split_body<true>(a); }

// Merge of the split records: out[h][d] = sum_s e^(m_s - M) acc_s[d] /
// sum_s e^(m_s - M) l_s, M = max_s m_s.  Grid heads, 256 threads.
extern "C" __global__ void __launch_bounds__(256) lp_attn_combine(const AttnArgs a) {
    const int h = blockIdx.x;
    const float* base = dptr<const float>(a.scratch) + (size_t)h * a.scratch_stride;
    const int rec = a.out_dim + 2;
    float M = -INFINITY;
    for (int s = 0; s < a.splits; ++s) M = fmaxf(M, base[(size_t)s * rec]);
    float den = 0.0f;
    for (int s = 0; s < a.splits; ++s) {
        const float ms = base[(size_t)s * rec];
        if (ms != -INFINITY) den = __builtin_fmaf(expf(ms - M), base[(size_t)s * rec + 1], den);
    }
    for (int d = threadIdx.x; d < a.out_dim; d += 256) {
        float num = 0.0f;
        for (int s = 0; s < a.splits; ++s) {
            const float ms = base[(size_t)s * rec];
            if (ms != -INFINITY) num = __builtin_fmaf(expf(ms - M), base[(size_t)s * rec + 2 + d], num);
        }
        dptr<float>(a.out)[(size_t)h * a.out_dim + d] = num / den;
    }
}

// ---------------------------------------------------------------------------
// Batched MLA decode over bf16 latent caches (config 5), on MFMA.  Grid
// (splits, batch), 4 waves.  Split s of sequence b walks its positions in
// chunks of 64 cache rows with an online softmax over the chunks:
//   scores  S[h][r] = scale * q_h . row_r: v_mfma_f32_16x16x32_bf16 with
//           the query as A (heads as M; its fp32 values split into bf16
//           hi + lo, two MFMAs per step, so the query keeps 16 significant
//           bits) and 16 cache rows per wave as B, loaded as 16-byte row
//           pieces straight into registers (the next chunk's loads are in
//           flight while this chunk's softmax and context are computed);
//   softmax per head over the chunk, the running max and sum rescaled;
//   context ctx[h][d] += sum_r p[h][r] row_r[d]: the same MFMA with the
//           probabilities (hi + lo) as A and the chunk as B (each wave a
//           quarter of the c_dim columns): the rows go to LDS as they are
//           (one 16-byte store per lane and step during the score pass) and
//           the B operand comes back column-wise through the transposing
//           LDS read (ds_read_b64_tr_b16: each 16-lane group reads a 4-row x
//           16-column block, lane i receiving column i's four values).
// The cache rows are read once from HBM.  Each split ends with a partial
// record {max[16], sum[16], acc[16][c_dim]}; lp_mla_combine merges them.
// ---------------------------------------------------------------------------
namespace {

__device__ __forceinline__ uint32_t pack_bf16(uint32_t lo, uint32_t hi) { return lo | (hi << 16); }

typedef short v4i16_t __attribute__((ext_vector_type(4)));

// e^x for the batched MLA's softmax (x <= 0 there): the hardware base-2
// exponential of x log2(e), within a few ulp (the bf16 cache bounds the
// result's precision far below that); -inf gives 0.
__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// hi / lo bf16 images of eight fp32 values, element order = value order
__device__ __forceinline__ void split8(const float (&v)[8], uint4& hi, uint4& lo) {
    uint32_t h[8], l[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        h[i] = f32_to_bf16_rne(v[i]);
        l[i] = f32_to_bf16_rne(v[i] - bf16_to_f32(h[i]));
    }
    hi = make_uint4(pack_bf16(h[0], h[1]), pack_bf16(h[2], h[3]), pack_bf16(h[4], h[5]), pack_bf16(h[6], h[7]));
    lo = make_uint4(pack_bf16(l[0], l[1]), pack_bf16(l[2], l[3]), pack_bf16(l[4], l[5]), pack_bf16(l[6], l[7]));
}

__device__ __forceinline__ f32x4_t mfma_bf16(const uint4& a, const uint4& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

template <int STEPS>
__device__ __forceinline__ void mla_split_body(const MlaBatchArgs& a) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int QK = 32 * STEPS;
    const int b = blockIdx.y, sp = blockIdx.x;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const int n = lane & 15, kb = lane >> 4;
    const int H = a.heads, CD = a.c_dim;
    const int tpw = CD >> 6;  // 16-column tiles per wave (a quarter of c_dim)
    uint4* qhi = reinterpret_cast<uint4*>(lds);
    uint4* qlo = qhi + STEPS * 64;
    const int rsb = mla_row_bytes(CD);
    uint8_t* ct = lds + 2 * STEPS * 1024;  // the chunk's first c_dim columns: [kMlaRows][rsb]
    const uint32_t ct_addr = lds_addr_of(ct);
    float* sl = reinterpret_cast<float*>(ct + kMlaRows * rsb);  // [16][64]
    // a length past the cache is cut to the cache (rows beyond max_seq
    // belong to the next sequence, or to no allocation at all)
    const int seq = min(dptr<const int>(a.seq_lens)[b], a.max_seq);
    const int p0 = sp * a.span;
    const int p1 = min(seq, p0 + a.span);
    const int nchunks = p1 > p0 ? (p1 - p0 + kMlaRows - 1) / kMlaRows : 0;
    // the query's hi / lo images in A order: step j, lane (m, kb) holds
    // q[m][32 j + 8 kb .. + 7]; heads past H are zero
    // the sequence's valid rows through a raw buffer: rows past p1 read zero
    const uint64_t cb = a.cache + (uint64_t)b * a.cache_stride;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void*>(uniform_u64(cb)), (short)0,
        __builtin_amdgcn_readfirstlane(p1 > 0 ? p1 * QK * 2 : 0), kBufferWord3);
    auto load_chunk = [&](uint4 (&B)[STEPS], int c) {
        const int row = p0 + c * kMlaRows + 16 * wave + n;
        const uint32_t off = (uint32_t)row * (QK * 2) + 16u * (uint32_t)kb;
#pragma unroll
        for (int j = 0; j < STEPS; ++j)
            B[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(off + 64u * j), 0, 0));
    };
    float m_run = -INFINITY, l_run = 0.0f;  // head n (every kb lane holds the same)
    f32x4_t acc[kMlaMaxC / 64];
#pragma unroll
    for (int c = 0; c < kMlaMaxC / 64; ++c) acc[c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // one register buffer: a chunk's rows are dead once its scores are made,
    // so the next chunk's loads go into the same registers at that point
    auto chunk = [&](uint4 (&Bc)[STEPS], int c) {
        // scores of rows 16 wave + n; the chunk's first c_dim columns stored
        // row by row for the context pass
        f32x4_t s4 = {0.0f, 0.0f, 0.0f, 0.0f};
        const int rl = 16 * wave + n;
#pragma unroll
        for (int j = 0; j < STEPS; ++j) {
            s4 = mfma_bf16(qhi[j * 64 + lane], Bc[j], s4);
            s4 = mfma_bf16(qlo[j * 64 + lane], Bc[j], s4);
            const int col = 32 * j + 8 * kb;
            if (col < CD) *reinterpret_cast<uint4*>(ct + (size_t)rl * rsb + col * 2) = Bc[j];
        }
        if (c + 1 < nchunks) load_chunk(Bc, c + 1);
        const bool rvalid = p0 + c * kMlaRows + rl < p1;
#pragma unroll
        for (int v = 0; v < 4; ++v) sl[(4 * kb + v) * kMlaRows + rl] = rvalid ? s4[v] * a.scale : -INFINITY;
        __syncthreads();
        // online softmax: lane (head n, kb) takes rows 32 s + 8 kb + i
        float sv[16];
        float mx = -INFINITY;
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                sv[8 * s + i] = sl[n * kMlaRows + 32 * s + 8 * kb + i];
                mx = fmaxf(mx, sv[8 * s + i]);
            }
        mx = fmaxf(mx, shfl_xor(mx, 16));
        mx = fmaxf(mx, shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const bool none = m_new == -INFINITY;  // every row so far masked
        const float alpha = none ? 1.0f : exp_hw(m_run - m_new);
        float ps = 0.0f;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            sv[t] = none ? 0.0f : exp_hw(sv[t] - m_new);
            ps += sv[t];
        }
        ps += shfl_xor(ps, 16);
        ps += shfl_xor(ps, 32);
        l_run = __builtin_fmaf(l_run, alpha, ps);
        m_run = m_new;
        float av[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) av[v] = __shfl(alpha, 4 * kb + v, 64);
        uint4 phi[2], plo[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            float v8[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v8[i] = sv[8 * s + i];
            split8(v8, phi[s], plo[s]);
        }
        // context over this wave's columns: lane (n, kb) needs rows
        // 32 s + 8 kb .. + 7 of column n; lane i of group kb points the
        // transposing read at row 32 s + 8 kb + i / 4, columns 4 (i % 4) .. + 3
        // of the 16-column tile (and 4 rows further for the second half)
        const int li = lane & 15;
#pragma unroll
        for (int t = 0; t < kMlaMaxC / 64; ++t) {
            if (t < tpw) {  // uniform
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[t][v] *= av[v];
                const int col0 = wave * (CD >> 2) + 16 * t;
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const uint32_t pa = ct_addr + (uint32_t)((32 * s + 8 * kb + (li >> 2)) * rsb) +
                                        (uint32_t)((col0 + 4 * (li & 3)) * 2);
                    const v4i16_t r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        reinterpret_cast<__attribute__((address_space(3))) v4i16_t*>((uintptr_t)pa));
                    const v4i16_t r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        reinterpret_cast<__attribute__((address_space(3))) v4i16_t*>((uintptr_t)(pa + 4u * rsb)));
                    const uint4 bt = make_uint4(pack_bf16((uint16_t)r0[0], (uint16_t)r0[1]),
                                                pack_bf16((uint16_t)r0[2], (uint16_t)r0[3]),
                                                pack_bf16((uint16_t)r1[0], (uint16_t)r1[1]),
                                                pack_bf16((uint16_t)r1[2], (uint16_t)r1[3]));
                    acc[t] = mfma_bf16(phi[s], bt, acc[t]);
                    acc[t] = mfma_bf16(plo[s], bt, acc[t]);
                }
            }
        }
        __syncthreads();  // the chunk's LDS is free for the next one
    };
    // the query's loads first, then the first chunk's rows: the loads retire
    // in order, so the query images are made while the rows are in flight
    uint4 B0[STEPS];
    {
        constexpr int kUnits = (STEPS * 64 + 255) / 256;  // query pieces per thread
        const uint64_t q = a.q + (uint64_t)b * H * QK * 4;
        float4 v4[kUnits][2];
#pragma unroll
        for (int r = 0; r < kUnits; ++r) {
            const int u = tid + 256 * r, j = u >> 6, l = u & 63, m = l & 15, k8 = l >> 4;
            v4[r][0] = v4[r][1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (u < STEPS * 64 && m < H) {
                const LP_GLOBAL float4* src = gptr<float4>(q + ((uint64_t)m * QK + 32 * j + 8 * k8) * 4);
                v4[r][0] = src[0];
                v4[r][1] = src[1];
            }
        }
        if (nchunks > 0) load_chunk(B0, 0);
#pragma unroll
        for (int r = 0; r < kUnits; ++r) {
            const int u = tid + 256 * r;
            if (u < STEPS * 64) {
                const float v[8] = {v4[r][0].x, v4[r][0].y, v4[r][0].z, v4[r][0].w,
                                    v4[r][1].x, v4[r][1].y, v4[r][1].z, v4[r][1].w};
                split8(v, qhi[u], qlo[u]);
            }
        }
    }
    __syncthreads();  // the query images
    for (int c = 0; c < nchunks; ++c) chunk(B0, c);
    // the partial record
    float* part = dptr<float>(a.part) + ((size_t)b * a.splits + sp) * mla_part_floats(CD);
    if (wave == 0 && lane < 16) {
        part[lane] = m_run;
        part[16 + lane] = l_run;
    }
#pragma unroll
    for (int t = 0; t < kMlaMaxC / 64; ++t) {
        if (t < tpw) {
            const int col = wave * (CD >> 2) + 16 * t + n;
#pragma unroll
            for (int v = 0; v < 4; ++v) part[32 + (size_t)(4 * kb + v) * CD + col] = acc[t][v];
        }
    }
}

}  // namespace

extern "C" __global__ void __launch_bounds__(256) lp_mla_split(const MlaBatchArgs a) {
    switch (a.qk_dim >> 5) {
        case 3: mla_split_body<3>(a); break;
        case 4: mla_split_body<4>(a); break;
        case 6: mla_split_body<6>(a); break;
        case 8: mla_split_body<8>(a); break;
        case 12: mla_split_body<12>(a); break;
        case 16: mla_split_body<16>(a); break;
        case 18: mla_split_body<18>(a); break;
        case 20: mla_split_body<20>(a); break;
        default: break;  // the host admits only these widths
    }
}

// ctx[b][h][d] from the splits' records.  Grid (heads, batch, c_dim / 64),
// 256 threads: the weights e^(m_s - M) / sum_s e^(m_s - M) l_s go to LDS once
// per workgroup, then thread (column d, group g) sums the splits s = g, g + 4,
// ... of its column (four loads in flight per step) and the four groups'
// sums meet in LDS.
extern "C" __global__ void __launch_bounds__(256) lp_mla_combine(const MlaBatchArgs a) {
    __shared__ float wsh[kMlaMaxSplits];
    __shared__ float red[4];
    __shared__ float part_sum[4][64];
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int CD = a.c_dim, PF = mla_part_floats(CD);
    const float* base = dptr<const float>(a.part) + (size_t)b * a.splits * PF;
    const float ms = tid < a.splits ? base[(size_t)tid * PF + h] : -INFINITY;
    const float ls = tid < a.splits ? base[(size_t)tid * PF + 16 + h] : 0.0f;
    const float M = block_max(ms, red);
    const float w = ms == -INFINITY ? 0.0f : expf(ms - M);
    const float den = block_sum(w * ls, red);
    if (tid < a.splits) wsh[tid] = w / den;
    __syncthreads();
    const int d = blockIdx.z * 64 + (tid & 63), g = tid >> 6;
    const float* col = base + 32 + (size_t)h * CD + d;
    float num = 0.0f;
    int s = g;
    for (; s + 12 < a.splits; s += 16) {
        const float v0 = col[(size_t)s * PF], v1 = col[(size_t)(s + 4) * PF];
        const float v2 = col[(size_t)(s + 8) * PF], v3 = col[(size_t)(s + 12) * PF];
        num = __builtin_fmaf(wsh[s], v0, num);
        num = __builtin_fmaf(wsh[s + 4], v1, num);
        num = __builtin_fmaf(wsh[s + 8], v2, num);
        num = __builtin_fmaf(wsh[s + 12], v3, num);
    }
    for (; s < a.splits; s += 4) num = __builtin_fmaf(wsh[s], col[(size_t)s * PF], num);
    part_sum[g][tid & 63] = num;
    __syncthreads();
    if (g == 0)
        dptr<float>(a.ctx)[((size_t)b * a.heads + h) * CD + d] =
            (part_sum[0][tid] + part_sum[1][tid]) + (part_sum[2][tid] + part_sum[3][tid]);
}
