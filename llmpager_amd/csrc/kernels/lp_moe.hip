// gfx950 kernels of the fused MoE layer: router GEMV, softmax / sigmoid
// top-k, token->expert dispatch, grouped q4 expert projections and the
// pick-order combine into the residual stream.
//
// Reference flow being replaced (one layer): decode.rs:303-342 (single token)
// and decode.rs:469-531 (multi-token union), kimi.rs:725-779 (sigmoid gating).
#include "lp_device.h"

using namespace lp;
using namespace lpk;

namespace {

template <typename T>
__device__ __forceinline__ T* dptr(uint64_t a) {
    return reinterpret_cast<T*>(a);
}

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// Order-preserving map of a finite float onto uint32 (larger float, larger key).
__device__ __forceinline__ uint32_t ordered_key(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// IEEE binary32 division, correctly rounded (the compiler's fdiv sequence:
// div_scale, a reciprocal refined by fused multiply-adds, div_fmas, div_fixup).
__device__ __forceinline__ float div_rn(float a, float b) { return a / b; }

// Data handed between workgroups of one launch: stores that write through to
// agent scope (sc1) and loads that read at agent scope, so that a relaxed
// arrival counter orders them without an L2 write-back or invalidate.
template <typename T>
__device__ __forceinline__ void store_agent(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void store_agent(LP_GLOBAL T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T load_agent(const LP_GLOBAL T* p) {
    return __hip_atomic_load(const_cast<LP_GLOBAL T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// ---------------------------------------------------------------------------
// Router GEMV: logits[t][e] = W_r[e, :] . x[t, :] (bf16 x f32, fp32 FMAs) in the
// canonical order: lane l takes 8-column chunks l, l+64, ... with fused
// multiply-adds, then a butterfly over the 64 lanes.  One wave per expert row,
// kRouterTokBlock tokens per wave.  Grid (ceil(E/4), ceil(T/8)).  With
// make_xf the workgroups of a token block also write those tokens' fragment
// images (one token per workgroup, round robin), which the grouped gate/up
// kernel copies straight into LDS.
// ---------------------------------------------------------------------------
namespace {

// Token t's digit image (the grouped kernels' A operand) from its row staged
// in LDS, by the whole workgroup: the four threads of a sub-group take eight
// columns each, share the sub-group's largest magnitude and their sum of xq
// by quad permutations (exact: a maximum and an integer sum), and write their
// eight columns' digits, which are contiguous in operand order (even columns,
// then odd).  The same bytes as write_dimage_group.
__device__ __forceinline__ void write_dimage_lds(const RouteArgs& a, int t, const float* row) {
    const int H = a.L.hidden, ng = H >> 5, ngp = frag_ngp(H);
    uint8_t* img = dptr<uint8_t>(a.W.xd) + (size_t)t * dimage_bytes(H);
    for (int u = threadIdx.x; u < 4 * ngp; u += blockDim.x) {  // whole quads together
        const int g = u >> 2, d = u & 3;
        float v[8];
        if (g < ng) {
            const float4 f0 = *reinterpret_cast<const float4*>(row + g * 32 + d * 8);
            const float4 f1 = *reinterpret_cast<const float4*>(row + g * 32 + d * 8 + 4);
            v[0] = f0.x; v[1] = f0.y; v[2] = f0.z; v[3] = f0.w;
            v[4] = f1.x; v[5] = f1.y; v[6] = f1.z; v[7] = f1.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = 0.0f;
        }
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
        m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xb1, 0xf, 0xf, false)));
        m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4e, 0xf, 0xf, false)));
        const bool live = m >= kDigitMin;
        const float inv = live ? 32639.0f / m : 0.0f;
        int hi[8], lo[8], sum = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) sum += digit_split(v[i], inv, hi[i], lo[i]);
        sum += __builtin_amdgcn_update_dpp(0, sum, 0xb1, 0xf, 0xf, false);
        sum += __builtin_amdgcn_update_dpp(0, sum, 0x4e, 0xf, 0xf, false);
        // columns 8d + {0, 2, 4, 6}, then 8d + {1, 3, 5, 7}
        *reinterpret_cast<uint2*>(img + (size_t)g * 32 + d * 8) =
            make_uint2(pack_i8x4(hi[0], hi[2], hi[4], hi[6]), pack_i8x4(hi[1], hi[3], hi[5], hi[7]));
        *reinterpret_cast<uint2*>(img + (size_t)ngp * 32 + (size_t)g * 32 + d * 8) =
            make_uint2(pack_i8x4(lo[0], lo[2], lo[4], lo[6]), pack_i8x4(lo[1], lo[3], lo[5], lo[7]));
        if (d == 0) {
            reinterpret_cast<int2*>(img + dimage_seed_off(ngp))[g] = make_int2(0, -8 * sum);
            reinterpret_cast<float*>(img + dimage_sigma_off(ngp))[g] = live ? m / 32639.0f : 0.0f;
        }
    }
}

// Token t's images from its row in memory, by the whole workgroup.
__device__ __forceinline__ void write_image(const RouteArgs& a, int t) {
    const int H = a.L.hidden;
    const float* row = dptr<const float>(a.x) + (size_t)t * H;
    if (a.make_xf & kImgDigits) {
        uint8_t* img = dptr<uint8_t>(a.W.xd) + (size_t)t * dimage_bytes(H);
        for (int g = threadIdx.x; g < frag_ngp(H); g += blockDim.x) write_dimage_group(row, H, g, img);
    }
    if (a.make_xf & kImgF16)
        write_h16_image(row, H, dptr<uint8_t>(a.W.xf) + (size_t)t * himage_bytes(H), dptr<int>(a.W.xexp) + t);
}

// Token t's images from its row staged in LDS.
__device__ __forceinline__ void write_images_lds(const RouteArgs& a, int t, const float* row) {
    if (a.make_xf & kImgDigits) write_dimage_lds(a, t, row);
    if (a.make_xf & kImgF16)
        write_h16_image(row, a.L.hidden, dptr<uint8_t>(a.W.xf) + (size_t)t * himage_bytes(a.L.hidden),
                        dptr<int>(a.W.xexp) + t);
}


// v + v[lane ^ o] for o = 32, 16, ..., 1 in turn (the router's butterfly):
// lane swaps for 32 and 16, a row rotation for 8, a swizzle for 4 and quad
// permutations for 2 and 1.  Each step adds the same two values as the
// shuffle form, so the result is bit-identical to it.
__device__ __forceinline__ float butterfly_sum(float v) {
    const auto a32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a32[0]) + __uint_as_float(a32[1]);
    const auto a16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a16[0]) + __uint_as_float(a16[1]);
    v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));  // row_ror:8
    v = v + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x101f));                      // xor 4
    v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, false));   // quad [2,3,0,1]
    v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, false));   // quad [1,0,3,2]
    return v;
}

// butterfly_sum over N independent values, step by step for all of them so
// that the steps' latencies overlap.
template <int N>
__device__ __forceinline__ void butterfly_sum_n(float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const auto a32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i]), false, false);
        v[i] = __uint_as_float(a32[0]) + __uint_as_float(a32[1]);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const auto a16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i]), false, false);
        v[i] = __uint_as_float(a16[0]) + __uint_as_float(a16[1]);
    }
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] = v[i] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[i]), 0x128, 0xf, 0xf, false));
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = v[i] + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v[i]), 0x101f));
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] = v[i] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[i]), 0x4e, 0xf, 0xf, false));
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] = v[i] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[i]), 0xb1, 0xf, 0xf, false));
}

// Logits of expert e for tokens t0 .. t0 + nt - 1 (nt <= kRouterTokBlock) by
// the calling wave.
__device__ __forceinline__ void router_dot(const RouteArgs& a, int e, int t0, int nt) {
    const int lane = lane_id();
    const int E = a.L.experts, H = a.L.hidden;
    const uint16_t* w = dptr<const uint16_t>(a.L.router_w) + (size_t)e * H;
    const float* x = dptr<const float>(a.x) + (size_t)t0 * H;
    float acc[kRouterTokBlock];
#pragma unroll
    for (int t = 0; t < kRouterTokBlock; ++t) acc[t] = 0.0f;
    const int chunks = H >> 3;
    for (int ch = lane; ch < chunks; ch += 64) {
        const uint4 wv = *reinterpret_cast<const uint4*>(w + ch * 8);
        const float wf[8] = {bf16_to_f32(wv.x & 0xffffu), bf16_to_f32(wv.x >> 16),
                             bf16_to_f32(wv.y & 0xffffu), bf16_to_f32(wv.y >> 16),
                             bf16_to_f32(wv.z & 0xffffu), bf16_to_f32(wv.z >> 16),
                             bf16_to_f32(wv.w & 0xffffu), bf16_to_f32(wv.w >> 16)};
#pragma unroll
        for (int t = 0; t < kRouterTokBlock; ++t) {
            if (t < nt) {
                const float4 xa = *reinterpret_cast<const float4*>(x + (size_t)t * H + ch * 8);
                const float4 xb = *reinterpret_cast<const float4*>(x + (size_t)t * H + ch * 8 + 4);
                float v = acc[t];
                v = __builtin_fmaf(wf[0], xa.x, v);
                v = __builtin_fmaf(wf[1], xa.y, v);
                v = __builtin_fmaf(wf[2], xa.z, v);
                v = __builtin_fmaf(wf[3], xa.w, v);
                v = __builtin_fmaf(wf[4], xb.x, v);
                v = __builtin_fmaf(wf[5], xb.y, v);
                v = __builtin_fmaf(wf[6], xb.z, v);
                v = __builtin_fmaf(wf[7], xb.w, v);
                acc[t] = v;
            }
        }
    }
    float* logits = dptr<float>(a.W.logits);
#pragma unroll
    for (int t = 0; t < kRouterTokBlock; ++t) {
        float v = acc[t];
        for (int o = 32; o >= 1; o >>= 1) v += shfl_xor(v, o);
        if (lane == 0 && t < nt) store_agent(&logits[(size_t)(t0 + t) * E + e], v);
    }
}

// Logits of experts e0 .. e0 + 8 * kRouteEPW - 1 (kRouteEPW per wave) for
// tokens t0 .. t0 + nt - 1 by the workgroup of 8 waves, in the same canonical
// order as router_dot.  The token rows are staged in LDS (xs, kRouteXLds
// bytes), as many as fit at a time, so that each is read from memory once per
// workgroup; each lane keeps its weight chunks of its experts in registers.

__device__ __forceinline__ void router_block(const RouteArgs& a, float* xs, int e0, int t0, int nt) {
    constexpr int CB = 4;  // weight chunks per lane loaded at once
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    const int E = a.L.experts, H = a.L.hidden;
    const int chunks = H >> 3;
    const int tb = min(kRouterTokBlock, kRouteXLds / (H * 4));
    LP_GLOBAL float* logits = gptr_w<float>(a.W.logits);
    int ew[kRouteEPW];
#pragma unroll
    for (int j = 0; j < kRouteEPW; ++j) ew[j] = min(e0 + wave * kRouteEPW + j, E - 1);
    for (int tt = 0; tt < nt; tt += tb) {
        const int nb = min(tb, nt - tt);
        float acc[kRouteEPW][kRouterTokBlock];
#pragma unroll
        for (int j = 0; j < kRouteEPW; ++j)
#pragma unroll
            for (int t = 0; t < kRouterTokBlock; ++t) acc[j][t] = 0.0f;
        for (int c0 = 0; c0 * 64 < chunks; c0 += CB) {
            // this batch's weight chunks of the wave's experts: in flight
            // together (and, for the first batch, with the staged rows)
            uint4 wv[kRouteEPW][CB];
#pragma unroll
            for (int j = 0; j < kRouteEPW; ++j)
#pragma unroll
                for (int c = 0; c < CB; ++c) {
                    const int ch = lane + 64 * (c0 + c);
                    wv[j][c] = make_uint4(0, 0, 0, 0);
                    if (ch < chunks)
                        wv[j][c] = *reinterpret_cast<const LP_GLOBAL uint4*>(gptr<uint16_t>(a.L.router_w) +
                                                                            (size_t)ew[j] * H + ch * 8);
                }
            if (c0 == 0) {
                __syncthreads();  // the previous sub-block's rows are consumed
                // every load of the staging in flight at once (up to
                // kRouteXLds / 16 / 512 per thread), then the LDS stores
                constexpr int XU = kRouteXLds / 16 / 512;
                const LP_GLOBAL float4* xg = gptr<float4>(a.x) + (size_t)(t0 + tt) * (H >> 2);
                const int n4 = nb * (H >> 2);
                float4 xr[XU];
#pragma unroll
                for (int u = 0; u < XU; ++u) {
                    const int i = (int)threadIdx.x + 512 * u;
                    xr[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    if (i < n4) xr[u] = xg[i];
                }
#pragma unroll
                for (int u = 0; u < XU; ++u) {
                    const int i = (int)threadIdx.x + 512 * u;
                    if (i < n4) reinterpret_cast<float4*>(xs)[i] = xr[u];
                }
                __syncthreads();
            }
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                const int ch = lane + 64 * (c0 + c);
                if (ch >= chunks) break;
                float wf[kRouteEPW][8];
#pragma unroll
                for (int j = 0; j < kRouteEPW; ++j) {
                    const uint4 w4 = wv[j][c];
                    wf[j][0] = bf16_to_f32(w4.x & 0xffffu);
                    wf[j][1] = bf16_to_f32(w4.x >> 16);
                    wf[j][2] = bf16_to_f32(w4.y & 0xffffu);
                    wf[j][3] = bf16_to_f32(w4.y >> 16);
                    wf[j][4] = bf16_to_f32(w4.z & 0xffffu);
                    wf[j][5] = bf16_to_f32(w4.z >> 16);
                    wf[j][6] = bf16_to_f32(w4.w & 0xffffu);
                    wf[j][7] = bf16_to_f32(w4.w >> 16);
                }
                // each staged row chunk is read once and serves every expert
#pragma unroll
                for (int t = 0; t < kRouterTokBlock; ++t) {
                    if (t < nb) {
                        const float4 xa = *reinterpret_cast<const float4*>(xs + (size_t)t * H + ch * 8);
                        const float4 xb = *reinterpret_cast<const float4*>(xs + (size_t)t * H + ch * 8 + 4);
#pragma unroll
                        for (int j = 0; j < kRouteEPW; ++j) {
                            float v = acc[j][t];
                            v = __builtin_fmaf(wf[j][0], xa.x, v);
                            v = __builtin_fmaf(wf[j][1], xa.y, v);
                            v = __builtin_fmaf(wf[j][2], xa.z, v);
                            v = __builtin_fmaf(wf[j][3], xa.w, v);
                            v = __builtin_fmaf(wf[j][4], xb.x, v);
                            v = __builtin_fmaf(wf[j][5], xb.y, v);
                            v = __builtin_fmaf(wf[j][6], xb.z, v);
                            v = __builtin_fmaf(wf[j][7], xb.w, v);
                            acc[j][t] = v;
                        }
                    }
                }
            }
        }
        float red[kRouteEPW * kRouterTokBlock];
#pragma unroll
        for (int j = 0; j < kRouteEPW; ++j)
#pragma unroll
            for (int t = 0; t < kRouterTokBlock; ++t) red[j * kRouterTokBlock + t] = acc[j][t];
        butterfly_sum_n(red);
#pragma unroll
        for (int j = 0; j < kRouteEPW; ++j) {
            const int e = e0 + wave * kRouteEPW + j;
#pragma unroll
            for (int t = 0; t < kRouterTokBlock; ++t)
                if (lane == 0 && e < E && t < nb)
                    store_agent(&logits[(size_t)(t0 + tt + t) * E + e], red[j * kRouterTokBlock + t]);
        }
    }
}

__device__ __forceinline__ void router_rows(const RouteArgs& a) {
    const int wave = threadIdx.x >> 6;
    const int e = blockIdx.x * 4 + wave;
    const int t0 = blockIdx.y * kRouterTokBlock;
    const int nt = min(kRouterTokBlock, a.T - t0);
    if (a.make_xf)
        for (int t = t0 + (int)blockIdx.x; t < t0 + nt; t += gridDim.x) write_image(a, t);
    if (e < a.L.experts) router_dot(a, e, t0, nt);
}

}  // namespace

extern "C" __global__ void __launch_bounds__(256) lp_moe_router(const RouteArgs a) { router_rows(a); }

// Images of x alone (callers that route from their own logits, and the
// large-batch router): one wave per token, lane l converting sub-groups l,
// l + 64, ... (digits) or 16-byte words l, l + 64, ... (fp16, after the row's
// largest magnitude), and W.xexp[t].  Grid (ceil(T / 4)), 256 threads.
extern "C" __global__ void __launch_bounds__(256) lp_moe_ximage(const RouteArgs a) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.T) return;
    const int H = a.L.hidden, lane = lane_id();
    const float* row = dptr<const float>(a.x) + (size_t)t * H;
    if (a.make_xf & kImgDigits) {
        uint8_t* img = dptr<uint8_t>(a.W.xd) + (size_t)t * dimage_bytes(H);
        for (int g = lane; g < frag_ngp(H); g += 64) write_dimage_group(row, H, g, img);
    }
    if (a.make_xf & kImgF16) {
        const int e = h16_exp(row_absmax_wave(row, H, lane, 64));
        write_h16_words(row, H, e, dptr<uint8_t>(a.W.xf) + (size_t)t * himage_bytes(H), lane, 64);
        if (lane == 0) dptr<int>(a.W.xexp)[t] = e;
    }
}

// ---------------------------------------------------------------------------
// Top-k gating, one wave per token.  Grid ceil(T/4) x 256.
//   softmax (decode.rs:734-749): m = max; e_i = expf(v_i - m); z = sum e_i in
//     id order; p_i = e_i / z; stable sort by p descending (ties: lower id);
//     first k; optional renormalisation by the in-order sum of the picks.
//   sigmoid (kimi.rs:1155-1186): s_i = 1/(1+expf(-v_i)); rank by s_i + bias_i
//     (stable, descending); weights s of the picks, renormalised if asked and
//     the sum is > 0, times routed_scaling; picks below min_weight dropped.
// expf is glibc's (lp_expf.h); every f32 operation is the reference's, in its
// order, so ids, order and weights match the host path bit for bit.
// ---------------------------------------------------------------------------
namespace {

// Top-k of token t by the calling wave, PER candidates per lane (expert
// i = lane + 64 q); sv is the wave's LDS row (kMaxExperts floats).  The
// in-order sum of the softmax: the exponentials go to sv and every lane
// reads them back (broadcast reads) and folds them in id order, a chain of
// adds on registers.  The k winners, already in the stable descending order,
// come one per round (select_rounds) on the ordered keys of p_i = e_i / z
// (sigmoid: of s_i + bias_i).  Ranking by e_i instead, while z is folded,
// would differ where two different e_i divide to one p_i; overlapping the two
// chains and checking for such ties after cost as much as it saved.  Pick r
// lands in lane r, which then finishes it.
template <int NR, int PER>
__device__ __forceinline__ int select_rounds(uint32_t (&key)[PER]) {
    // live keys are >= 1; 0 marks no expert (and a taken one).  Round r: the
    // largest key left, the lowest id holding it (ids lane + 64 q: the first
    // non-empty ballot, its lowest lane), that key cleared; lane r keeps the
    // id.  Rounds past the live keys leave garbage in lanes past them.
    const int lane = lane_id();
    int pk = -1;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        uint32_t mx = key[0];
#pragma unroll
        for (int q = 1; q < PER; ++q) mx = key[q] > mx ? key[q] : mx;
        mx = wave_max_u32(mx);
        int win = -1;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const uint64_t b = __ballot(key[q] == mx);
            if (win < 0 && b != 0ull) win = 64 * q + (int)__builtin_ctzll(b);  // uniform
        }
#pragma unroll
        for (int q = 0; q < PER; ++q)
            if (lane + 64 * q == win) key[q] = 0u;
        if (lane == r) pk = win;
    }
    return pk;
}

template <int PER>
__device__ __forceinline__ void topk_token(const RouteArgs& a, int t, float* sv, int* ids_l, int* cnt_l) {
    const int lane = lane_id();
    const int E = a.L.experts, k = a.L.top_k;
    const LP_GLOBAL float* lg = gptr<float>(a.W.logits) + (size_t)t * E;
    const uint64_t tabv = exp2tab_lane();  // glibc's 2^(i/32) table, one entry per lane
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    constexpr int kZ = 8;  // float4 reads of sv in flight per fold batch
    uint32_t key[PER];
    float val[PER], v[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        const int i = lane + 64 * q;
        v[q] = i < E ? load_agent(lg + i) : 0.0f;
        key[q] = 0u;
        val[q] = 0.0f;
    }
    const int n = k < E ? k : E;
    // the value of expert p (its lane's val); every lane must call it
    auto pick_val = [&](int p) {
        float pv = 0.0f;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const float vq = __int_as_float(__builtin_amdgcn_ds_bpermute((p & 63) * 4, __float_as_int(val[q])));
            if ((p >> 6) == q) pv = vq;
        }
        return pv;
    };
    if (a.L.gating == 0) {
        uint32_t mk = 0u;  // max over the ordered keys = the largest logit (f32::MIN start)
#pragma unroll
        for (int q = 0; q < PER; ++q)
            if (lane + 64 * q < E) mk = mk > ordered_key(v[q]) ? mk : ordered_key(v[q]);
        mk = wave_max_u32(mk);
        float m = __uint_as_float((mk & 0x80000000u) ? (mk & 0x7fffffffu) : ~mk);
        m = fmaxf(m, -3.40282347e+38f);
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const float ex = expf_glibc_wave(v[q] - m, tabv);  // every lane takes part
            v[q] = lane + 64 * q < E ? ex : 0.0f;
        }
        // z = e_0 + e_1 + ... in id order, from -0.0 (the reference's fold).
        // sv holds e_i for i < 64 PER (+0.0 past E); folding those trailing
        // zeros changes nothing once the first term is in (z is then >= +0,
        // and z + 0 = z), so the fold runs over whole batches of 4 kZ.
#pragma unroll
        for (int q = 0; q < PER; ++q) sv[lane + 64 * q] = v[q];
        wave_sync_lds();
        float z = -0.0f;
        const int nz = PER <= 2 ? 64 * PER : (E + 4 * kZ - 1) / (4 * kZ) * (4 * kZ);
        for (int c = 0; c < nz; c += 4 * kZ) {
            float4 f[kZ];
#pragma unroll
            for (int u = 0; u < kZ; ++u) f[u] = *reinterpret_cast<const float4*>(sv + c + 4 * u);
#pragma unroll
            for (int u = 0; u < kZ; ++u) {
                z = z + f[u].x;
                z = z + f[u].y;
                z = z + f[u].z;
                z = z + f[u].w;
            }
        }
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            if (lane + 64 * q < E) {
                val[q] = div_rn(v[q], z);
                key[q] = ordered_key(val[q]);
            }
        }
    } else {
        const LP_GLOBAL float* bias = gptr<float>(a.L.router_bias);
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = lane + 64 * q;
            const float ex = expf_glibc_wave(-v[q], tabv);  // every lane takes part
            if (i < E) {
                const float d = 1.0f + ex;
                val[q] = div_rn(1.0f, d);
                key[q] = ordered_key((val[q] + bias[i]) + 0.0f);  // -0 ranks equal to +0
            }
        }
    }
    // live keys are >= 1 (ordered_key(-inf) = 0x007fffff), n at most the live keys
    const int pk = n <= 8 ? select_rounds<8>(key) : select_rounds<kMaxTopK>(key);
    // pick j in lane j (its value fetched from the winner's lane); the sum of
    // the picks in pick order, from -0.0
    const bool inn = lane < n;
    const float pv = pick_val(pk);  // every lane: the permutes read from any lane
    const int my_pick = inn ? pk : -1;
    const float my_val = inn ? pv : 0.0f;
    float s = -0.0f;
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
        if (j >= n) break;  // uniform
        s = s + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_val), j));
    }
    float wj = my_val;
    bool keep = inn;
    if (a.L.gating == 0) {
        if (a.L.renorm) wj = div_rn(my_val, s);
    } else {
        if (a.L.renorm && s > 0.0f) wj = div_rn(wj, s);
        wj = wj * a.L.routed_scaling;
        if (a.L.min_weight > 0.0f && !(wj >= a.L.min_weight)) keep = false;
    }
    // survivors keep pick order: pick j moves to slot (survivors before it),
    // the dropped ones after them, lanes n.. stay (a permutation again)
    const uint64_t km = __ballot(keep);
    const int kept = __popcll(km);
    int out_pick = my_pick;
    float out_w = wj;
    if (kept != n) {  // uniform
        const uint64_t nm = n >= 64 ? ~0ull : ((1ull << n) - 1ull);
        const int dst = keep ? __popcll(km & below) : (inn ? kept + __popcll(~km & nm & below) : lane);
        out_pick = __builtin_amdgcn_ds_permute(dst * 4, my_pick);
        out_w = __int_as_float(__builtin_amdgcn_ds_permute(dst * 4, __float_as_int(wj)));
    }
    if (lane < k) {
        const int id = lane < kept ? out_pick : -1;
        store_agent(gptr_w<int>(a.W.ids) + (size_t)t * k + lane, id);
        store_agent(gptr_w<float>(a.W.wts) + (size_t)t * k + lane, lane < kept ? out_w : 0.0f);
        if (ids_l) ids_l[t * k + lane] = id;
    }
    if (lane == 0) {
        store_agent(gptr_w<int>(a.W.cnt) + t, kept);
        if (cnt_l) cnt_l[t] = kept;
    }
}

// Top-k of token t with the candidate count per lane the expert count needs
// (PMAX 2: at most 128 experts, the only form compiled); ids_l / cnt_l (may
// be null) receive LDS copies of the picks.
template <int PMAX = kMaxExperts / 64>
__device__ __forceinline__ void topk_any(const RouteArgs& a, int t, float* sv, int* ids_l = nullptr,
                                         int* cnt_l = nullptr) {
    if (PMAX == 2 || a.L.experts <= 128)
        topk_token<2>(a, t, sv, ids_l, cnt_l);
    else if (a.L.experts <= 256)
        topk_token<4>(a, t, sv, ids_l, cnt_l);
    else
        topk_token<kMaxExperts / 64>(a, t, sv, ids_l, cnt_l);
}

}  // namespace

extern "C" __global__ void __launch_bounds__(256) lp_moe_topk(const RouteArgs a) {
    __shared__ float sh_v[4][kMaxExperts];
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t < a.T) topk_any(a, t, sh_v[threadIdx.x >> 6]);
}

// ---------------------------------------------------------------------------
// Dispatch (one workgroup of 256): the (t, j) picks stably grouped by expert
// id, then t ascending.  Writes group starts gs[E+1], perm[pos] = t*k + j,
// inv[t*k + j] = pos (-1 for unused pick slots), uniq[] (experts with picks,
// ascending), meta[0] = unique count (meta[1], the error flags, cleared), and
// the expert table et[u] for u < min(T*k, E) that the grouped kernels read
// (blob address through the slot table, positions, first kEntryToks tokens).
// Stability comes from ranking each pick by the tokens before it with the
// same expert (a 64-bit token mask per expert; every caller has T <= 64).
// ---------------------------------------------------------------------------
namespace {

// Exclusive scan of one int per thread over the workgroup (<= 16 waves).
__device__ __forceinline__ int block_excl_scan(int v, int* sh, int* total) {
    const int lane = lane_id(), wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int x = wave_incl_scan(v);
    if (lane == 63) sh[wave] = x;
    __syncthreads();
    int wbase = 0, tot = 0;
    for (int w = 0; w < nw; ++w) {
        wbase += w < wave ? sh[w] : 0;
        tot += sh[w];
    }
    *total = tot;
    __syncthreads();
    return wbase + x - v;
}

// LDS of dispatch_all, carved from one buffer so that the single-workgroup
// top-k + dispatch kernel can share it with its top-k phase: token masks
// (2 x E), group starts (E + 4), unique list (E), first tokens (E x
// kEntryToks), picks (kTopkDispatchMaxT x kMaxTopK), pick counts
// (kTopkDispatchMaxT), slot table (E) and 4 words.
constexpr int kDispatchSmem = 4 * (kMaxExperts * 2 + (kMaxExperts + 4) + kMaxExperts + kMaxExperts * kEntryToks +
                                   kTopkDispatchMaxT * (kMaxTopK + 1) + kMaxExperts + 4);
static_assert(kTopkDispatchMaxT <= 64, "dispatch_all ranks the tokens of one 64-bit mask");

// ids / cnt: the picks (global, or LDS copies from the same workgroup);
// slots: the slot table (global, or an LDS copy).
// The shared MLP's table (if the layer has one): every token, identity
// dispatch order, as shared_entries(T) entries of consecutive tokens (groups
// of 4 for decode batches, so the grouped kernels take it without token
// loops; one entry for larger batches).  Threads tid, tid + nth, ... of the
// caller write it.
__device__ __forceinline__ void write_shared_table(const RouteArgs& a, int tid, int nth) {
    if (!a.L.shared_blob) return;
    const int T = a.T, nv = shared_entries(T);
    const int per = nv == 1 ? T : kEntryToks;
    for (int t = tid; t < T; t += nth) gptr_w<int>(a.W.sh_perm)[t] = t;
    for (int v = tid; v < nv; v += nth) {
        ExpertEntry x;
        x.blob = a.L.shared_blob;
        x.p0 = v * per;
        x.ntok = min(per, T - v * per);
#pragma unroll
        for (int q = 0; q < kEntryToks; ++q) x.tok[q] = q < x.ntok ? x.p0 + q : -1;
        gptr_w<ExpertEntry>(a.W.sh_et)[v] = x;
    }
}

// in_global: ids_in / cnt_in are the workspace's (written by other
// workgroups of this launch: read at agent scope), else LDS copies.
__device__ __forceinline__ void dispatch_all(const RouteArgs& a, uint8_t* sm, const int* ids_in,
                                             const int* cnt_in, const int* slots_in, bool in_global) {
    // T <= kTopkDispatchMaxT <= 64: expert e's picks are the set bits of
    // its token mask (a token picks an expert at most once), its count is
    // the mask's popcount and a pick's rank among them the bits below its
    // token; one thread per pick, four barriers.
    uint32_t* mlo = reinterpret_cast<uint32_t*>(sm);  // tokens 0..31
    uint32_t* mhi = mlo + kMaxExperts;                 // tokens 32..63
    int* gsl = reinterpret_cast<int*>(mhi + kMaxExperts);  // kMaxExperts + 1 used
    int* uniq_l = gsl + kMaxExperts + 4;
    int (*tokf)[kEntryToks] = reinterpret_cast<int (*)[kEntryToks]>(uniq_l + kMaxExperts);
    int* ids = uniq_l + kMaxExperts + kMaxExperts * kEntryToks;
    int* cnt = ids + kTopkDispatchMaxT * kMaxTopK;
    int* slots = cnt + kTopkDispatchMaxT;
    int* nu_l = slots + kMaxExperts;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const int nth = blockDim.x;
    const int E = a.L.experts, k = a.L.top_k, T = a.T, P = T * k;
    LP_GLOBAL int* perm = gptr_w<int>(a.W.perm);
    LP_GLOBAL int* inv = gptr_w<int>(a.W.inv);
    LP_GLOBAL int* meta = gptr_w<int>(a.W.meta);
    // the picks and the slot table in LDS (one round trip when they are in
    // memory), the masks and first tokens cleared
    for (int i = tid; i < P; i += nth) ids[i] = in_global ? load_agent(gptr<int>((uint64_t)ids_in) + i) : ids_in[i];
    for (int i = tid; i < T; i += nth) cnt[i] = in_global ? load_agent(gptr<int>((uint64_t)cnt_in) + i) : cnt_in[i];
    for (int e = tid; e < E; e += nth) {
        slots[e] = slots_in[e];
        mlo[e] = 0u;
        mhi[e] = 0u;
#pragma unroll
        for (int q = 0; q < kEntryToks; ++q) tokf[e][q] = -1;
    }
    __syncthreads();
    for (int p = tid; p < P; p += nth) {
        const int t = p / k, j = p - t * k;
        if (j < cnt[t]) atomicOr(t < 32 ? &mlo[ids[p]] : &mhi[ids[p]], 1u << (t & 31));
    }
    __syncthreads();
    // one wave: counts, their exclusive scan (group starts) and the unique
    // list, 64 experts a pass
    if (wave == 0) {
        const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        int run = 0, urun = 0;
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int e = e0 + lane;
            const int c = e < E ? __popc(mlo[e]) + __popc(mhi[e]) : 0;
            const int x = wave_incl_scan(c);
            const uint64_t f = __ballot(c > 0);
            if (e < E) gsl[e] = run + x - c;
            if (c > 0) uniq_l[urun + __popcll(f & below)] = e;
            run += __builtin_amdgcn_readlane(x, 63);
            urun += __popcll(f);
        }
        if (lane == 0) {
            gsl[E] = run;
            *nu_l = urun;
            meta[0] = urun;
            meta[1] = 0;
        }
    }
    __syncthreads();
    // each pick's position: its expert's start plus the tokens before it
    // with the same expert
    for (int p = tid; p < P; p += nth) {
        const int t = p / k, j = p - t * k;
        if (j < cnt[t]) {
            const int e = ids[p];
            const uint64_t m = (uint64_t)mlo[e] | ((uint64_t)mhi[e] << 32);
            const int rank = __popcll(m & ((1ull << t) - 1ull));
            const int pos = gsl[e] + rank;
            perm[pos] = p;
            inv[p] = pos;
            if (rank < kEntryToks) tokf[e][rank] = t;
        } else {
            inv[p] = -1;
        }
    }
    const int nu = *nu_l;
    LP_GLOBAL int* gs = gptr_w<int>(a.W.gs);
    for (int e = tid; e <= E; e += nth) gs[e] = gsl[e];
    LP_GLOBAL int* uniq = gptr_w<int>(a.W.uniq);
    for (int u = tid; u < nu; u += nth) uniq[u] = uniq_l[u];
    write_shared_table(a, tid, nth);
    __syncthreads();
    // the expert table for the grouped kernels
    LP_GLOBAL ExpertEntry* et = gptr_w<ExpertEntry>(a.W.et);
    const int maxu = min(P, E);
    for (int u = tid; u < maxu; u += nth) {
        ExpertEntry x;
        if (u < nu) {
            const int e = uniq_l[u];
            const int slot = slots[e];
            x.blob = slot >= 0 ? a.L.arena_base + (uint64_t)slot * a.L.slot_span : 0ull;
            x.p0 = gsl[e];
            x.ntok = gsl[e + 1] - gsl[e];
#pragma unroll
            for (int q = 0; q < kEntryToks; ++q) x.tok[q] = tokf[e][q];
        } else {
            x.blob = 0ull;
            x.p0 = 0;
            x.ntok = 0;
#pragma unroll
            for (int q = 0; q < kEntryToks; ++q) x.tok[q] = -1;
        }
        et[u] = x;
    }
}

// dispatch_all's tables for at most 64 picks (lane p: pick p = t k + j,
// valid when j < cnt[t]), by the waves of one workgroup and no barrier.
// Pick p's key is e * 64 + p (an id above every expert's for the others):
// its position in the expert-major order, stable by token as dispatch_all's,
// is the number of smaller keys.  The keys reach every lane of a wave
// through its scr (the wave's own 192 words of LDS: broadcast reads into
// registers), and wave 0 writes the sorted keys and tokens back to scr, so
// lane u reads position u's pick, whether it starts its expert's run, the run
// length (the next start, from a ballot) and the run's first tokens.  Waves
// w = 0 .. nw - 1 call it together: wave 0 writes every table but gs, which
// the other waves write, 64 entries each in turn (wave 0 too when alone).
__device__ __forceinline__ int below_count(const int* bk, int nb, int key) {
    // keys bk[0 .. 16 nb) (all >= 0) against key: how many are smaller
    int n = 0;
    for (int b = 0; b < nb; ++b) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int4 x = *reinterpret_cast<const int4*>(bk + 16 * b + 4 * i);
            n += (int)(((uint32_t)(x.x - key) >> 31) + ((uint32_t)(x.y - key) >> 31) +
                       ((uint32_t)(x.z - key) >> 31) + ((uint32_t)(x.w - key) >> 31));
        }
    }
    return n;
}

__device__ __forceinline__ void dispatch_keys(const RouteArgs& a, const int* ids_in, const int* cnt_in,
                                              const int* slots_in, int* scr, int w, int nw) {
    const int lane = lane_id();
    const int E = a.L.experts, k = a.L.top_k, T = a.T;
    const int P = T * k;  // <= 64
    const int t = lane / k, j = lane - t * k;
    const bool inb = lane < P;
    const int c = inb ? cnt_in[t] : 0;
    const bool valid = inb && j < c;
    const int e = valid ? ids_in[lane] : 0;
    constexpr int kNone = 0x7fffffff;
    const int key = valid ? (e << 6) | lane : kNone;
    scr[lane] = key;
    wave_sync_lds();
    const int nb = (P + 15) >> 4;  // blocks of 16 keys to compare
    if (w > 0 || nw == 1) {
        // gs[x] = valid picks with an expert id below x = keys below x * 64
        LP_GLOBAL int* gs = gptr_w<int>(a.W.gs);
        const int gw = nw == 1 ? 0 : w - 1, ng = nw == 1 ? 1 : nw - 1;
        for (int x0 = 64 * gw; x0 <= E; x0 += 64 * ng) {
            const int x = x0 + lane;
            const int below = below_count(scr, nb, x << 6);
            if (x <= E) gs[x] = below;
        }
        if (w > 0) return;
    }
    const int pos = below_count(scr, nb, key);
    const int nv = __popcll(__ballot(valid));
    if (valid) {
        scr[64 + pos] = key;
        scr[128 + pos] = t;
    }
    if (inb) gptr_w<int>(a.W.inv)[lane] = valid ? pos : -1;
    wave_sync_lds();
    // lane u: dispatch position u
    const int u = lane;
    const bool live = u < nv;
    const int ku = live ? scr[64 + u] : kNone;
    const int eu = ku >> 6;
    const int kp = u > 0 && live ? scr[64 + u - 1] : kNone;
    const bool first = live && (u == 0 || (kp >> 6) != eu);
    const uint64_t F = __ballot(first);
    const int U = __popcll(F);
    const uint64_t below = u == 0 ? 0ull : (~0ull >> (64 - u));
    const int uidx = __popcll(F & below);
    if (live) gptr_w<int>(a.W.perm)[u] = ku & 63;
    LP_GLOBAL ExpertEntry* et = gptr_w<ExpertEntry>(a.W.et);
    if (first) {
        const uint64_t later = F & ~below & ~(1ull << u);  // starts after u
        const int ntok = (later ? (int)__builtin_ctzll(later) : nv) - u;
        gptr_w<int>(a.W.uniq)[uidx] = eu;
        const int slot = slots_in[eu];
        ExpertEntry x;
        x.blob = slot >= 0 ? a.L.arena_base + (uint64_t)slot * a.L.slot_span : 0ull;
        x.p0 = u;
        x.ntok = ntok;
#pragma unroll
        for (int r = 0; r < kEntryToks; ++r) x.tok[r] = r < ntok ? scr[128 + u + r] : -1;
        et[uidx] = x;
    }
    const int maxu = min(P, E);
    if (lane >= U && lane < maxu) {
        ExpertEntry x;
        x.blob = 0ull;
        x.p0 = 0;
        x.ntok = 0;
#pragma unroll
        for (int r = 0; r < kEntryToks; ++r) x.tok[r] = -1;
        et[lane] = x;
    }
    if (lane == 0) {
        gptr_w<int>(a.W.meta)[0] = U;
        gptr_w<int>(a.W.meta)[1] = 0;
    }
    write_shared_table(a, lane, 64);
}

}  // namespace

// Dispatch of a medium batch after the multi-workgroup top-k: dispatch_all
// over the picks in memory, one workgroup of 256.
extern "C" __global__ void __launch_bounds__(256) lp_moe_dispatch(const RouteArgs a) {
    __shared__ __align__(16) uint8_t sm[kDispatchSmem];
    dispatch_all(a, sm, dptr<const int>(a.W.ids), dptr<const int>(a.W.cnt), dptr<const int>(a.L.slot_table), true);
}

// ---------------------------------------------------------------------------
// Dispatch of a large batch in three launches, with the single-workgroup
// dispatch_all's result: picks grouped by expert (ascending id), in token
// order within an expert (the order decode.rs:469-531 visits them).
//   count:   per block of kDispTok tokens, each expert's picks;
//   scan:    group starts, each block's first position per expert, the
//            unique list, the expert table and the expert -> entry map;
//   scatter: per block, each pick's rank among its expert's picks of the
//            block (earlier waves' counts plus the set bits below the lane in
//            the wave's 64-bit mask of that expert), added to the block's
//            first position.
// W.disp holds [nb][E] counts, then [nb][E] first positions, then [E] entry
// indices (nb = ceil(T / kDispTok)).
// ---------------------------------------------------------------------------

// Grid ceil(T / kDispTok), kDispTok threads.
extern "C" __global__ void __launch_bounds__(kDispTok) lp_moe_disp_count(const RouteArgs a) {
    __shared__ int h[kMaxExperts];
    const int E = a.L.experts, k = a.L.top_k, T = a.T;
    const int tid = threadIdx.x, b = blockIdx.x;
    for (int e = tid; e < E; e += kDispTok) h[e] = 0;
    __syncthreads();
    const int t = b * kDispTok + tid;
    if (t < T) {
        const int c = dptr<const int>(a.W.cnt)[t];
        const int* ids = dptr<const int>(a.W.ids) + (size_t)t * k;
        for (int j = 0; j < c; ++j) atomicAdd(&h[ids[j]], 1);
    }
    __syncthreads();
    int* cnt = dptr<int>(a.W.disp) + (size_t)b * E;
    for (int e = tid; e < E; e += kDispTok) cnt[e] = h[e];
}

// One workgroup of 1024 threads: thread e takes expert e.
extern "C" __global__ void __launch_bounds__(1024) lp_moe_disp_scan(const RouteArgs a) {
    __shared__ int scan_sh[16];
    const int E = a.L.experts, k = a.L.top_k, T = a.T;
    const int nb = (T + kDispTok - 1) / kDispTok;
    const int tid = threadIdx.x;
    const int* cnt = dptr<const int>(a.W.disp);
    int* first = dptr<int>(a.W.disp) + (size_t)nb * E;
    int* uidx = first + (size_t)nb * E;
    int tot = 0;
    if (tid < E)
        for (int b = 0; b < nb; ++b) tot += cnt[(size_t)b * E + tid];
    int total, nu;
    const int g0 = block_excl_scan(tot, scan_sh, &total);
    const int u = block_excl_scan(tot > 0 ? 1 : 0, scan_sh, &nu);
    ExpertEntry* et = dptr<ExpertEntry>(a.W.et);
    if (tid < E) {
        dptr<int>(a.W.gs)[tid] = g0;
        int o = g0;
        for (int b = 0; b < nb; ++b) {
            first[(size_t)b * E + tid] = o;
            o += cnt[(size_t)b * E + tid];
        }
        uidx[tid] = tot > 0 ? u : -1;
        if (tot > 0) {
            dptr<int>(a.W.uniq)[u] = tid;
            const int slot = dptr<const int>(a.L.slot_table)[tid];
            ExpertEntry x;
            x.blob = slot >= 0 ? a.L.arena_base + (uint64_t)slot * a.L.slot_span : 0ull;
            x.p0 = g0;
            x.ntok = tot;
#pragma unroll
            for (int q = 0; q < kEntryToks; ++q) x.tok[q] = -1;  // the scatter fills the first ones
            et[u] = x;
        }
    }
    if (tid == 0) {
        dptr<int>(a.W.gs)[E] = total;
        dptr<int>(a.W.meta)[0] = nu;
        dptr<int>(a.W.meta)[1] = 0;
    }
    // entries past the unique ones are cleared, as dispatch_all does
    const int maxu = min(T * k, E);
    for (int v = nu + tid; v < maxu; v += blockDim.x) {
        ExpertEntry x;
        x.blob = 0ull;
        x.p0 = 0;
        x.ntok = 0;
#pragma unroll
        for (int q = 0; q < kEntryToks; ++q) x.tok[q] = -1;
        et[v] = x;
    }
    write_shared_table(a, tid, blockDim.x);
}

// Grid ceil(T / kDispTok), kDispTok threads (wave w: tokens 64 w .. of the block).
extern "C" __global__ void __launch_bounds__(kDispTok) lp_moe_disp_scatter(const RouteArgs a) {
    constexpr int W = kDispTok / 64;
    __shared__ uint32_t mlo[W][kMaxExperts], mhi[W][kMaxExperts];
    __shared__ int woff[W][kMaxExperts];
    const int E = a.L.experts, k = a.L.top_k, T = a.T;
    const int nb = (T + kDispTok - 1) / kDispTok;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6, b = blockIdx.x;
    for (int i = tid; i < W * E; i += kDispTok) {
        mlo[i / E][i % E] = 0u;
        mhi[i / E][i % E] = 0u;
    }
    __syncthreads();
    const int t = b * kDispTok + tid;
    const int c = t < T ? dptr<const int>(a.W.cnt)[t] : 0;
    const int* ids = dptr<const int>(a.W.ids) + (size_t)t * k;
    for (int j = 0; j < c; ++j) atomicOr(lane < 32 ? &mlo[wave][ids[j]] : &mhi[wave][ids[j]], 1u << (lane & 31));
    __syncthreads();
    const int* first = dptr<const int>(a.W.disp) + (size_t)nb * E + (size_t)b * E;
    for (int e = tid; e < E; e += kDispTok) {
        int o = first[e];
#pragma unroll
        for (int w = 0; w < W; ++w) {
            woff[w][e] = o;
            o += __popc(mlo[w][e]) + __popc(mhi[w][e]);
        }
    }
    __syncthreads();
    if (t >= T) return;
    int* perm = dptr<int>(a.W.perm);
    int* inv = dptr<int>(a.W.inv);
    const int* gs = dptr<const int>(a.W.gs);
    const int* uidx = first + (size_t)(nb - b) * E;  // [E] after the first positions
    ExpertEntry* et = dptr<ExpertEntry>(a.W.et);
    const uint64_t below = (1ull << lane) - 1ull;
    for (int j = 0; j < k; ++j) {
        if (j < c) {
            const int e = ids[j];
            const uint64_t mask = (uint64_t)mlo[wave][e] | ((uint64_t)mhi[wave][e] << 32);
            const int pos = woff[wave][e] + __popcll(mask & below);
            perm[pos] = t * k + j;
            inv[t * k + j] = pos;
            const int r = pos - gs[e];
            if (r < kEntryToks) et[uidx[e]].tok[r] = t;
        } else {
            inv[t * k + j] = -1;
        }
    }
}

// Re-resolve the expert table's blob addresses through the layer's current
// slot table: the paged flow routes first, asks the pager for the picked
// experts (whose slots the pager then writes into the table), and only then
// runs the expert kernels.  One workgroup.
extern "C" __global__ void __launch_bounds__(256) lp_moe_resolve(const RouteArgs a) {
    const int maxu = min(a.T * a.L.top_k, a.L.experts);
    const int nu = dptr<const int>(a.W.meta)[0];
    const int* uniq = dptr<const int>(a.W.uniq);
    const int* slots = dptr<const int>(a.L.slot_table);
    ExpertEntry* et = dptr<ExpertEntry>(a.W.et);
    for (int u = threadIdx.x; u < maxu && u < nu; u += blockDim.x) {
        const int slot = slots[uniq[u]];
        et[u].blob = slot >= 0 ? a.L.arena_base + (uint64_t)slot * a.L.slot_span : 0ull;
    }
}

// ---------------------------------------------------------------------------
// Top-k and dispatch in one workgroup of 1024 threads, for the smallest
// batches (the host uses it for T <= kTopkFusedMaxT, at most one token per
// wave): wave w ranks token w, then the whole workgroup builds the dispatch
// tables.  One launch less than lp_moe_topk + lp_moe_dispatch; past one token
// per wave the top-k on a single CU costs more than the extra launch.
// ---------------------------------------------------------------------------
extern "C" __global__ void __launch_bounds__(1024) lp_moe_topk_dispatch(const RouteArgs a) {
    constexpr int kTopkLds = 16 * kMaxExperts * 4;
    __shared__ __align__(16) uint8_t sm[kDispatchSmem > kTopkLds ? kDispatchSmem : kTopkLds];
    __shared__ int ids_l[kTopkFusedMaxT * kMaxTopK];
    __shared__ int cnt_l[kTopkFusedMaxT];
    __shared__ int slots_l[kMaxExperts];
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    // the slot table comes in while the picks are made
    const int* slots = dptr<const int>(a.L.slot_table);
    for (int e = threadIdx.x; e < a.L.experts; e += blockDim.x) slots_l[e] = slots[e];
    float* sv = reinterpret_cast<float*>(sm) + wave * kMaxExperts;
    for (int t = wave; t < a.T; t += nw) topk_any(a, t, sv, ids_l, cnt_l);
    __syncthreads();
    dispatch_all(a, sm, ids_l, cnt_l, slots_l, false);
}

// ---------------------------------------------------------------------------
// Routing of a decode-sized batch (T <= kTopkDispatchMaxT) in one launch:
// router logits, top-k and dispatch.  Grid (ceil(E/(8 kRouteEPW)), ceil(T/8)),
// 512 threads: workgroup (g, b) computes the logits of experts
// 8 kRouteEPW g .. (kRouteEPW per wave, the router GEMV's canonical order)
// for the tokens of block b (8b .. 8b+7).  The last workgroup of block b to
// finish (an arrival counter) ranks the block's tokens, one per wave, while
// the others write the block's fragment images (make_xf); the last block to
// finish ranking builds the dispatch tables.  Logits and picks cross between
// workgroups as agent-scope stores and loads (arrival_order); the last
// arrival resets its counter, so every launch finds them zero.
// ---------------------------------------------------------------------------
namespace {

// Add one arrival at *cnt; returns (in every thread) the workgroup's arrival
// order, n - 1 for the last, which also resets the counter.  Every thread of
// the workgroup must call it.  What one workgroup hands to another across an
// arrival (logits, then picks) is written with agent-scope stores (they
// write through this XCD's L2) and read with agent-scope loads, so each wave
// only waits until its own stores have completed before the barrier and a
// relaxed counter orders the rest: no L2 write-back or invalidate (each of
// those costs microseconds).
__device__ __forceinline__ int arrival_order(int* cnt, int n, int* flag) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's stores have completed at agent scope
    __syncthreads();
    if (threadIdx.x == 0) {
        const int o = atomicAdd(cnt, 1);
        if (o == n - 1) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = o;
    }
    __syncthreads();
    return *flag;
}

__device__ __forceinline__ bool last_arrival(int* cnt, int n, int* flag) {
    return arrival_order(cnt, n, flag) == n - 1;
}

}  // namespace

template <int PMAX>
__device__ __forceinline__ void route_fused_body(const RouteArgs& a) {
    constexpr int kTopkLds = 8 * kMaxExperts * 4;
    __shared__ __align__(16) uint8_t sm[kDispatchSmem > kTopkLds ? kDispatchSmem : kTopkLds];
    __shared__ __align__(16) float xs[kRouteXLds / 4];
    __shared__ int slots_l[kMaxExperts];
    __shared__ int ids_l[kRouterTokBlock * kMaxTopK];  // one token block's picks
    __shared__ int cnt_l[kRouterTokBlock];
    __shared__ int flag;
    static_assert(kMaxExperts <= 2 * 512, "two slot-table entries per thread");
    const int wave = threadIdx.x >> 6, tid = threadIdx.x;
    const int b = blockIdx.y, t0 = b * a.tok_block;
    const int nt = min(a.tok_block, a.T - t0);
    // the slot table comes in with the router weights (every workgroup:
    // which one dispatches is known only at the end)
    const int E = a.L.experts;
    const LP_GLOBAL int* st = gptr<int>(a.L.slot_table);
    const int sl0 = tid < E ? st[tid] : 0;
    const int sl1 = tid + 512 < E ? st[tid + 512] : 0;
    router_block(a, xs, blockIdx.x * 8 * kRouteEPW, t0, nt);
    if (tid < E) slots_l[tid] = sl0;
    if (tid + 512 < E) slots_l[tid + 512] = sl1;
    // The images are for the expert kernels only.  The workgroups that are
    // not the last of their block to arrive write them, shared by arrival
    // order, after arriving: the last one, which goes on to rank the block,
    // writes none (unless it is alone), so no image store or release waits
    // on the ranking's path.  From the rows still staged in LDS when the
    // whole block fits there.
    auto images = [&](int first, int step) {
        if (!a.make_xf) return;
        const bool staged = nt * a.L.hidden * 4 <= kRouteXLds;
        for (int t = first; t < nt; t += step) {
            if (staged)
                write_images_lds(a, t0 + t, xs + (size_t)t * a.L.hidden);
            else
                write_image(a, t0 + t);
        }
    };
    int* cnt = dptr<int>(a.sync);
    const int order = arrival_order(cnt + kSyncStride * b, gridDim.x, &flag);
    if (order != (int)gridDim.x - 1) {
        images(order, gridDim.x - 1);
        return;
    }
    if (gridDim.x == 1) images(0, 1);
    // one token block: the picks also go to LDS (token t = wave)
    const bool one = gridDim.y == 1;
    if (wave < nt)
        topk_any<PMAX>(a, t0 + wave, reinterpret_cast<float*>(sm) + wave * kMaxExperts, one ? ids_l : nullptr,
                 one ? cnt_l : nullptr);
    if (one) {
        // ranked by this workgroup: no second arrival, and the tables come
        // from LDS alone; up to kDispatchKeysMaxPicks picks are placed by
        // sort keys, more by dispatch_all
        __syncthreads();
        if (a.T * a.L.top_k <= kDispatchKeysMaxPicks) {
            dispatch_keys(a, ids_l, cnt_l, slots_l, reinterpret_cast<int*>(sm) + wave * kMaxExperts, wave,
                          (int)(blockDim.x >> 6));
        } else {
            dispatch_all(a, sm, ids_l, cnt_l, slots_l, false);
        }
        return;
    }
    if (!last_arrival(cnt + kSyncStride * 16, gridDim.y, &flag)) return;
    dispatch_all(a, sm, dptr<const int>(a.W.ids), dptr<const int>(a.W.cnt), slots_l, true);
}

extern "C" __global__ void __launch_bounds__(512) lp_moe_route_fused(const RouteArgs a) { route_fused_body<kMaxExperts / 64>(a); }

// The same for at most 128 experts: only that top-k form compiled, a kernel
// of about half the code (the whole fused kernel outgrows the instruction
// cache).
extern "C" __global__ void __launch_bounds__(512) lp_moe_route_fused128(const RouteArgs a) { route_fused_body<2>(a); }

// ---------------------------------------------------------------------------
// Grouped expert projections.  A workgroup of W waves takes one work item =
// (routed expert u, run of rows); every wave owns 16-row tiles of that run and
// the workgroup stages the expert's tokens into shared LDS fragments, up to
// kMaxPairs token pairs at a time.  The item's only dependent load is its
// expert-table entry; the first chunk of weights is in flight while the
// fragments are staged, and each dequantised weight word serves every staged
// token pair.  Small per-wave state keeps several workgroups resident per CU
// so one item's latency hides behind another's work.
//   gate/up: act[pos][r] = silu(gate_e . x_t)[r] * (up_e . x_t)[r], r < I
//   down:    y[pos][r]   = (down_e . act[pos])[r], r < H
// pos = dispatch position of the (token, pick) pair.  An expert without a
// slot raises kErrMissingExpert in meta[1] and its outputs are zero.
// ---------------------------------------------------------------------------
namespace {

__device__ __forceinline__ ExpertEntry entry_at(uint64_t table, int u) {
    const LP_GLOBAL uint4* p = gptr<uint4>(table + (uint64_t)u * sizeof(ExpertEntry));
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

__device__ __forceinline__ ExpertEntry entry_of(const GroupedArgs& a, int u) {
    const LP_GLOBAL uint4* p = gptr<uint4>(a.W.et + (uint64_t)u * sizeof(ExpertEntry));
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

// Token of the expert's i-th (token, pick) pair: from the entry for the first
// kEntryToks (no dependent load), else through the dispatch permutation.
// Token i < kEntryToks of the entry, from the entry alone.
__device__ __forceinline__ int entry_tok(const ExpertEntry& x, int i) {
    static_assert(kEntryToks == 4, "select chain below");
    return i == 0 ? x.tok[0] : i == 1 ? x.tok[1] : i == 2 ? x.tok[2] : x.tok[3];
}

__device__ __forceinline__ int pair_token(const ExpertEntry& x, int i, const int* perm, int k) {
    static_assert(kEntryToks == 4, "select chain below");
    return i == 0 ? x.tok[0] : i == 1 ? x.tok[1] : i == 2 ? x.tok[2] : i == 3 ? x.tok[3] : perm[x.p0 + i] / k;
}

// Share of workgroup blockIdx.x when the grid's workgroups are handed to
// the 8 XCDs round-robin: consecutive shares go to one XCD, when the grid is
// a multiple of 8.  (The one-shot grouped kernels keep blockIdx order: their
// work items of one entry on one XCD made a config-5 layer of 16 tokens
// 122 us against 98.6.)
__device__ __forceinline__ int xcd_item() {
    const int G = (int)gridDim.x, b = (int)blockIdx.x;
    return (G & 7) == 0 ? (b & 7) * (G >> 3) + (b >> 3) : b;
}

__device__ __forceinline__ void missing_expert(const GroupedArgs& a, const ExpertEntry& x, float* out,
                                               int stride, int rows, int row_lo, int row_hi) {
    if (threadIdx.x == 0) atomicOr(dptr<int>(a.W.meta) + 1, kErrMissingExpert);
    for (int p = 0; p < x.ntok; ++p)
        for (int r = row_lo + (int)threadIdx.x; r < row_hi && r < rows; r += blockDim.x)
            out[(size_t)(x.p0 + p) * stride + r] = 0.0f;
}

// gate/up MFMAs for one staged token group of P pairs, then SiLU * up into
// act.  GU (gate, up) holds the tile's first chunk on entry.  A tile of one
// chunk (ONE: S <= NS) is straight-line code and simply stays in registers
// for the next token group.  Longer tiles load each further chunk right
// after the previous one's MFMAs and, when another token group follows
// (`reload`), the first chunk again before the epilogue, so that latency
// overlaps the stores and the next group's image copy.
template <int P, int NS, bool ONE, int RS, bool SL>
__device__ __forceinline__ void gateup_group(const Frags& F, WRegs<NS, SL> (&GU)[2], const WTile<RS>& TG,
                                             const WTile<RS>& TU, int I, int n0, int S, int t0,
                                             int nt, int p0, bool reload, float* act) {
    const int np = (nt + 1) >> 1;
    float acc[2][P][2];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int p = 0; p < P; ++p) acc[m][p][0] = acc[m][p][1] = 0.0f;
    if constexpr (ONE) {
        opaque(GU[0]);
        opaque(GU[1]);
        ABase B[P];
#pragma unroll
        for (int p = 0; p < P; ++p) B[p] = abase(F, p, 0);
        wmma(GU, B, S, np, acc);
    } else {
#pragma nounroll
        for (int c0 = 0;;) {
            ABase B[P];
#pragma unroll
            for (int p = 0; p < P; ++p) B[p] = abase(F, p, c0);
            wmma(GU, B, S - c0, np, acc);
            c0 += NS;
            if (c0 >= S) break;
            wload(GU[0], TG, c0);
            wload(GU[1], TU, c0);
        }
        if (reload) {
            wload(GU[0], TG, 0);
            wload(GU[1], TU, 0);
        }
    }
    const int lane = lane_id();
    const int row = n0 + (lane & 15);
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const float g0 = tile_reduce(acc[0][p][0]), g1 = tile_reduce(acc[0][p][1]);
        const float u0 = tile_reduce(acc[1][p][0]), u1 = tile_reduce(acc[1][p][1]);
        const int t = 2 * p + (lane >> 4);  // within the group
        if (row < I && lane < 32 && t < nt) {
            const float g = lane < 16 ? g0 : g1;
            const float u = lane < 16 ? u0 : u1;
            act[(size_t)(p0 + t0 + t) * I + row] = g / (1.0f + expf(-g)) * u;
        }
    }
}

// Bytes of a wave's LDS scale window for one tile (WRegs SL).
template <int NS>
__host__ __device__ constexpr int scale_window_bytes() { return 64 * 2 * window_steps<NS>(); }

template <int NS, bool ONE, int RS, bool SL>
__device__ __forceinline__ void gateup_body(const GroupedArgs& a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const LayerView& L = a.L;
    const int H = L.hidden, I = L.inter, k = L.top_k;
    const int wave = threadIdx.x >> 6, W = blockDim.x >> 6;
    const int run = kTileRows * W;
    const int chunks = (I + run - 1) / run;
    const int u = blockIdx.x / chunks;
    const int chunk = blockIdx.x - u * chunks;
    const ExpertEntry x = entry_of(a, u);
    if (x.ntok == 0) return;
    float* act = dptr<float>(a.W.act);
    if (x.blob == 0) {
        missing_expert(a, x, act, I, I, chunk * run, chunk * run + run);
        return;
    }
    const int S = tile_steps(H);
    const int n0 = chunk * run + kTileRows * wave;
    const Frags F = frags_at(lds, H);
    const WTile<RS> TG = wtile<RS>(x.blob + L.gate_off, I, H, n0);
    const WTile<RS> TU = wtile<RS>(x.blob + L.up_off, I, H, n0);
    const int* perm = dptr<const int>(a.W.perm);
    const uint64_t xf = a.W.xd;
    const uint64_t ib = (uint64_t)dimage_bytes(H);
    const int cap = min(kMaxPairs, a.pairs_cap);
    // The first token group's images (tokens from the entry: no lookup) are
    // copied first, the weights loaded after them; one wait then covers both
    // and their latencies overlap.
    zero_block(F, threadIdx.x, blockDim.x);
    issue_images(F, min(2 * cap, x.ntok), [&](int t) { return xf + (uint64_t)entry_tok(x, t) * ib; });
    // the wave's two scale windows follow the fragment area (SL)
    const uint32_t swin = lds_addr_of(lds) + (uint32_t)frag_lds_bytes(H, a.pairs_cap) +
                          (uint32_t)(2 * wave * scale_window_bytes<NS>());
    WRegs<NS, SL> GU[2];
    wload(GU[0], TG, 0, swin);
    wload(GU[1], TU, 0, swin + scale_window_bytes<NS>());
    for (int tb = 0; tb < x.ntok; tb += 2 * cap) {
        const int nt = min(2 * cap, x.ntok - tb);
        const bool reload = tb + nt < x.ntok;
        if (tb == 0) {
            __builtin_amdgcn_s_waitcnt(0);  // the copies (and the weights) have landed
        } else {
            __syncthreads();
            load_images(F, nt, [&](int t) { return xf + (uint64_t)pair_token(x, tb + t, perm, k) * ib; });
        }
        __syncthreads();
        gateup_group<kMaxPairs, NS, ONE, RS, SL>(F, GU, TG, TU, I, n0, S, tb, nt, x.p0, reload, act);
    }
}

// ---------------------------------------------------------------------------
// Balanced gate/up for decode batches (lp_moe_gateup_bal).  One workgroup of
// kBalWaves waves per CU.  Work is cut into units of 8 rows of gate plus the
// same 8 rows of up over the whole of K (one MFMA tile: lanes n < 8 carry gate
// row r0 + n, lanes n >= 8 up row r0 + n - 8), for each token group
// (routed expert, up to kBalToks = 4 of its tokens), in blocks of up to
// kBalGroups groups of one expert ordered row unit by row unit (BalPlan).
// Every workgroup takes an equal contiguous range of the V * R units (V
// groups, R = ceil(I / 8)); with V no larger than the grid a range touches
// at most two blocks, whose tokens' images are staged once, into two LDS
// slots.  Each wave then
// walks its units (every W-th of the range, W waves), one at a time: a
// unit's loads, then its MFMAs, the workgroup's waves overlapping one
// another's loads and math (a second register buffer, the next unit's
// weights in flight during the current one's MFMAs, measured slower: the
// extra loads only lengthen the memory system's queues).  Loads and stores
// are issued unconditionally (a missing expert's unit reads a zero-size
// buffer, a lane with nothing to store writes past the end of act, which
// the hardware drops).  No barrier after the start.
// ---------------------------------------------------------------------------

// The merged gate/up tile of rows [r0, r0 + 8) of an expert blob; `valid`
// false gives a tile whose nibble loads read zeros and whose scale-window
// copies (SL) read the first bytes at `dummy`.
template <int RS>
__device__ __forceinline__ WTile<RS> wtile_gu(uint64_t blob, bool valid, uint64_t dummy, uint32_t goff,
                                              uint32_t uoff, int rows, int cols, int r0) {
    const int lane = lane_id();
    const int n = lane & 15, kb = lane >> 4;
    const uint32_t ng = (uint32_t)cols >> 5, gpr = ng >> RS;
    const uint32_t sbytes = (uint32_t)rows * gpr * 2;
    const uint32_t rbytes = sbytes + (uint32_t)rows * ng * 16;
    const uint32_t row = (uint32_t)min(r0 + (n & 7), rows - 1);
    const uint32_t off = n < 8 ? goff : uoff;
    // blob, valid and the record count are uniform over the wave; saying so
    // keeps the resource in SGPRs (no per-lane loop around each load)
    const uint64_t base = uniform_u64(valid ? blob : dummy);
    const int nrec = __builtin_amdgcn_readfirstlane(valid ? (int)(max(goff, uoff) + rbytes) : 0);
    WTile<RS> T;
    T.rsrc = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(base), (short)0, nrec, kBufferWord3);
    T.base = base;
    T.dofs = off + sbytes + (row * ng + kb) * 16;
    T.sofs = valid ? off + (row * gpr + (kb >> RS)) * 2 : 2u * (uint32_t)(kb >> RS);
    T.lastok = (ng & 3) == 0 || kb < (int)(ng & 3);
    return T;
}

// The workgroup's share of a balanced launch.  An entry's tokens form
// ceil(ntok / kBalToks) token groups ("virtual experts", numbered by a prefix
// sum over the expert table); runs of up to kBalGroups groups of one entry
// form a block whose units are ordered row-major: unit i of the block is row
// unit i / g of token group i % g (g groups), so the units that read the same
// weight rows for different token groups are neighbours, taken by
// neighbouring waves of one workgroup at the same time, and the rows come
// from HBM once.  The workgroup takes the contiguous range [lo, hi) of the
// V * R units; with V no larger than the grid a range is at most R units
// long and a block at least R, so it touches at most two blocks, whose
// tokens are staged into two LDS slots of kBalGroups * kBalPairs pairs.
// Returns false for an empty range (the whole workgroup).  The LDS meta area
// follows the fragments of `cols`-wide rows (bal_meta_off).
struct BalPlan {
    int lo, hi, nslot;
    ExpertEntry x[2];  // the slots' entries (slot 1 repeats slot 0 when the range has one block)
    int start[2];      // first unit of the slot's block
    int tg0[2];        // first token group of the block (tokens kBalToks tg0 ..)
    int gq[2];         // token groups in the block (1..kBalGroups)
    int ns[2];         // tokens in the block (1..kBalToks kBalGroups)
    int sh[2];         // the block is the shared MLP's (an entry of W.sh_et)

    // Unit un (uniform): slot s, row unit u, token group gl within the block.
    __device__ __forceinline__ void unit(int un, int& s, int& u, int& gl) const {
        s = nslot == 2 && un >= start[1] ? 1 : 0;
        const int i = un - (s ? start[1] : start[0]);
        const int g = s ? gq[1] : gq[0];
        u = g == 3 ? (i * 43691) >> 17 : i >> (g >> 1);  // i / g for g in 1..4, i < 2^16
        gl = i - u * g;
    }
};
static_assert(kBalGroups <= 4, "BalPlan::unit divides by at most 4");

// The routed entries (R units per token group) and, with SH and a.sh_maxu,
// the shared MLP's entries after them (Rs units per group: its own width).
template <bool SH = false>
__device__ __forceinline__ bool bal_plan(const GroupedArgs& a, uint8_t* lds, int cols, int R, int Rs, BalPlan& P) {
    const int tid = (int)threadIdx.x, lane = lane_id(), wave = tid >> 6, W = (int)(blockDim.x >> 6);
    const int maxu = a.maxu, nent = SH ? a.maxu + a.sh_maxu : a.maxu;
    int* tot = reinterpret_cast<int*>(lds + bal_meta_off(cols));  // [kBalWaves] wave totals
    int* sl = tot + kBalWaves;  // [2][3]: entry, first token group, first unit of the blocks of lo and hi - 1
    ExpertEntry* ent = reinterpret_cast<ExpertEntry*>(lds + bal_meta_off(cols) + 128);
    if (tid < 6) sl[tid] = 0;
    int ng = 0;
    const int Re = !SH || tid < maxu ? R : Rs;  // this entry's units per token group
    if (tid < nent) {
        const ExpertEntry x = !SH || tid < maxu ? entry_of(a, tid) : entry_at(a.W.sh_et, tid - maxu);
        ent[tid] = x;
        ng = (x.ntok + kBalToks - 1) / kBalToks;
    }
    const int inc = wave_incl_scan(ng * Re);  // units, prefix-summed
    if (lane == 63) tot[wave] = inc;
    __syncthreads();
    int before = 0, N = 0;
    for (int w = 0; w < W; ++w) {
        const int t = tot[w];
        before += w < wave ? t : 0;
        N += t;
    }
    const int u0 = before + inc - ng * Re;  // this entry's first unit
    // workgroups of one XCD take neighbouring shares
    const int b = xcd_item(), G = (int)gridDim.x;
    P.lo = (int)((long)N * b / G);
    P.hi = (int)((long)N * (b + 1) / G);
    if (P.lo >= P.hi) return false;
    if (tid < nent && ng > 0) {
        const int u1 = u0 + Re * ng;  // the entry's units
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int un = e == 0 ? P.lo : P.hi - 1;
            if (u0 <= un && un < u1) {
                const int q = (un - u0) / (Re * kBalGroups);
                sl[3 * e] = tid;
                sl[3 * e + 1] = q * kBalGroups;
                sl[3 * e + 2] = u0 + q * Re * kBalGroups;
            }
        }
    }
    __syncthreads();
    P.nslot = sl[2] != sl[5] ? 2 : 1;  // two blocks: their first units differ
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int q = s < P.nslot ? s : 0;
        P.x[s] = ent[sl[3 * q]];
        P.tg0[s] = sl[3 * q + 1];
        P.start[s] = sl[3 * q + 2];
        const int ngx = (P.x[s].ntok + kBalToks - 1) / kBalToks;
        P.gq[s] = min(kBalGroups, ngx - P.tg0[s]);
        P.ns[s] = min(kBalToks * kBalGroups, P.x[s].ntok - kBalToks * P.tg0[s]);
        P.sh[s] = SH && sl[3 * q] >= maxu;
    }
    return true;
}

// The MFMAs of one balanced unit of M weight tiles: np (1..kBalPairs,
// uniform) picks a straight-line form for exactly that many token pairs.
template <int NS, bool SL, int M>
__device__ __forceinline__ void bal_wmma(const WRegs<NS, SL> (&R)[M], const ABase (&B)[kBalPairs], int rem, int np,
                                         float (&acc)[M][kBalPairs][2]) {
    static_assert(kBalPairs == 2 || kBalPairs == 4, "one form per pair count");
    if constexpr (kBalPairs == 2) {
        if (np == 1) wmma<NS, SL, kBalPairs, M, 1>(R, B, rem, np, acc);
        else wmma<NS, SL, kBalPairs, M, 2>(R, B, rem, np, acc);
    } else {
        switch (np) {
            case 1: wmma<NS, SL, kBalPairs, M, 1>(R, B, rem, np, acc); break;
            case 2: wmma<NS, SL, kBalPairs, M, 2>(R, B, rem, np, acc); break;
            case 3: wmma<NS, SL, kBalPairs, M, 3>(R, B, rem, np, acc); break;
            default: wmma<NS, SL, kBalPairs, M, 4>(R, B, rem, np, acc); break;
        }
    }
}

// The token sums over K of a balanced tile's kBalPairs pairs (acc[p][h] =
// lane partials of token 2p + h): row r of X holds token quad_row_tok(r), row
// r of Y token 4 + quad_row_tok(r) (zero with two pairs).
__device__ __forceinline__ void bal_sums(const float (&acc)[kBalPairs][2], float& X, float& Y) {
    X = quad_rows(pair_rows(acc[0][0], acc[0][1]), pair_rows(acc[1][0], acc[1][1]));
    if constexpr (kBalPairs == 4)
        Y = quad_rows(pair_rows(acc[2][0], acc[2][1]), pair_rows(acc[3][0], acc[3][1]));
    else
        Y = 0.0f;
}

template <int NS, int RS, bool SL, bool SH = false>
__device__ __forceinline__ void gateup_bal_body(const GroupedArgs& a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const LayerView& L = a.L;
    const int H = L.hidden, I = L.inter, k = L.top_k;
    // the wave index said to be uniform: unit indices, slots and token counts
    // then live in SGPRs and the pair loop branches on them
    const int lane = lane_id(), wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int W = (int)(blockDim.x >> 6);
    const int R = (I + 7) >> 3;
    const int Ish = SH && a.sh_maxu ? L.shared_inter : I;  // the shared MLP's entries (SH) have their own width
    const Frags F = frags_at(lds, H);
    zero_block(F, threadIdx.x, blockDim.x);
    BalPlan P;
    if (!bal_plan<SH>(a, lds, H, R, (Ish + 7) >> 3, P)) return;
    const int lo = P.lo, hi = P.hi;
    // the two slots' blob, dispatch position and token count of the block,
    // and (a shared MLP block) its width, regions and act rows
    uint64_t sblob[2];
    int sp0[2], snt[2], sI[2];
    uint32_t sgo[2], suo[2];
    const uint64_t xf = a.W.xd, ib = (uint64_t)dimage_bytes(H);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const ExpertEntry x = P.x[s];
        const int tb = kBalToks * P.tg0[s];
        const bool sh = SH && P.sh[s] != 0;
        sblob[s] = x.blob;
        sp0[s] = x.p0 + tb;
        snt[s] = x.ntok - tb;
        sI[s] = sh ? Ish : I;
        sgo[s] = (uint32_t)(sh ? L.sh_gate_off : L.gate_off);
        suo[s] = (uint32_t)(sh ? L.sh_up_off : L.up_off);
        if (s < P.nslot) {
            Frags Fs = F;
            Fs.lds = F.lds + kBalGroups * kBalPairs * s * frag_pair_bytes(F.ngp);
            // shared entries hold consecutive tokens (all in tok[] for up to
            // kEntryToks; a routed entry's later ones through perm)
            const LP_GLOBAL int* perm = gptr<int>(sh ? a.W.sh_perm : a.W.perm);
            const int kk = sh ? 1 : k;
            issue_images(Fs, P.ns[s], [&](int t) {
                const int i = tb + t;
                const int tok = i < kEntryToks ? entry_tok(x, i) : perm[x.p0 + i] / kk;
                return xf + (uint64_t)tok * ib;
            });
        }
    }
    // this wave's units: lo + wave + W * j < hi
    const int J = hi - lo > wave ? (hi - lo - wave + W - 1) / W : 0;
    const int Sx = tile_steps(H);
    const uint64_t dummy = L.router_w;
    const uint32_t swin = lds_addr_of(lds) + (uint32_t)bal_win_off(H) +
                          (uint32_t)(wave * scale_window_bytes<NS>());
    LP_GLOBAL float* act = gptr_w<float>(a.W.act);
    auto load = [&](WRegs<NS, SL>& B, int j, uint32_t win) {
        int s, u, gl;
        P.unit(lo + wave + W * j, s, u, gl);
        const uint64_t blob = s == 0 ? sblob[0] : sblob[1];
        const bool valid = j < J && blob != 0;
        const WTile<RS> T = wtile_gu<RS>(blob, valid, dummy, s == 0 ? sgo[0] : sgo[1], s == 0 ? suo[0] : suo[1],
                                         s == 0 ? sI[0] : sI[1], H, 8 * u);
        wload(B, T, 0, win);
    };
    // act through a raw buffer: a lane with nothing to store writes at its end,
    // which the hardware drops, so every unit issues the same memory operations
    const uint32_t act_bytes = (uint32_t)a.T * (uint32_t)k * (uint32_t)I * 4u;
    const __amdgpu_buffer_rsrc_t act_rs =
        __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(a.W.act), (short)0, (int)act_bytes, kBufferWord3);
    const uint32_t sh_bytes = SH && a.sh_maxu ? (uint32_t)a.T * (uint32_t)Ish * 4u : 0u;
    const __amdgpu_buffer_rsrc_t sh_rs =
        __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(a.W.sh_act), (short)0, (int)sh_bytes, kBufferWord3);
    bool missing = false;
    auto compute = [&](const WRegs<NS, SL>& B, int j) {
        int s, ru, gl;
        P.unit(lo + wave + W * j, s, ru, gl);
        const int r0 = 8 * ru;
        const uint64_t qblob = s == 0 ? sblob[0] : sblob[1];
        const int qp0 = (s == 0 ? sp0[0] : sp0[1]) + kBalToks * gl;
        const int qnt = min(kBalToks, (s == 0 ? snt[0] : snt[1]) - kBalToks * gl);
        const int np = (qnt + 1) >> 1;
        missing |= qblob == 0;  // not resident: zero outputs, flag raised after the loop
        WRegs<NS, SL> Rm[1] = {B};
        if constexpr (SL) {
            // read the scale window only once B's first nibble load has landed,
            // and with it the window copies issued before that load
            uint32_t z;
            asm("v_and_b32 %0, 0, %1" : "=v"(z) : "v"(B.w[0].x));
            Rm[0].sbase += z;
        }
        float acc[1][kBalPairs][2];
#pragma unroll
        for (int p = 0; p < kBalPairs; ++p) acc[0][p][0] = acc[0][p][1] = 0.0f;
        ABase Bs[kBalPairs];
#pragma unroll
        for (int p = 0; p < kBalPairs; ++p) Bs[p] = abase(F, kBalPairs * (kBalGroups * s + gl) + p, 0);
        bal_wmma(Rm, Bs, Sx, np, acc);
        // the tokens' sums over K (bal_sums); in each row the gate of weight
        // row r0 + n sits in lane n < 8, its up in lane n + 8.  Lanes n < 8
        // finish X's tokens, lanes n >= 8 Y's (their gate brought over by a
        // rotation of the row by 8): one SiLU and one store per lane.
        float X, Y;
        bal_sums(acc[0], X, Y);
        const float rX = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(X), 0x128, 0xf, 0xf, false));
        const float rY = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(Y), 0x128, 0xf, 0xf, false));
        const bool hy = (lane & 15) >= 8;
        const float g = hy ? rY : X, u = hy ? Y : rX;
        const int t = (hy ? 4 : 0) + quad_row_tok(lane >> 4);
        const int row = r0 + (lane & 7);
        const float v = qblob == 0 ? 0.0f : g / (1.0f + expf(-g)) * u;
        const bool shb = SH && (s == 0 ? P.sh[0] : P.sh[1]) != 0;  // uniform
        const int Iq = shb ? Ish : I;
        const bool st = row < Iq && t < qnt;
        const uint32_t lim = shb ? sh_bytes : act_bytes;
        const uint32_t off = st ? ((uint32_t)(qp0 + t) * (uint32_t)Iq + (uint32_t)row) * 4u : lim;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), shb ? sh_rs : act_rs, (int)off, 0, 0);
    };
    WRegs<NS, SL> RA;
    load(RA, 0, swin);
    __builtin_amdgcn_s_waitcnt(0);  // images, seeds and the first unit have landed
    __syncthreads();
    for (int j = 0; j < J; ++j) {
        if (j > 0) load(RA, j, swin);
        compute(RA, j);
    }
    if (missing && lane == 0) atomicOr(gptr_w<int>(a.W.meta) + 1, kErrMissingExpert);
    __builtin_amdgcn_s_waitcnt(0);  // the last (past-the-end) unit's loads
}

// Balanced down for decode batches (lp_moe_down_bal): the plan of the
// balanced gate/up over units of 16 rows of down (all of K = inter), the
// slots' act rows staged as fragments, one unit at a time per wave as in the
// gate/up, and branch-free stores into y (a dropped one past its end).
template <int RS>
__device__ __forceinline__ WTile<RS> wtile_dn(uint64_t blob, bool valid, uint64_t dummy, uint32_t off, int rows,
                                              int cols, int r0) {
    const int lane = lane_id();
    const int n = lane & 15, kb = lane >> 4;
    const uint32_t ng = (uint32_t)cols >> 5, gpr = ng >> RS;
    const uint32_t sbytes = (uint32_t)rows * gpr * 2;
    const uint32_t rbytes = sbytes + (uint32_t)rows * ng * 16;
    const uint32_t row = (uint32_t)min(r0 + n, rows - 1);
    // blob, valid and the record count are uniform over the wave
    const uint64_t base = uniform_u64(valid ? blob + off : dummy);
    const int nrec = __builtin_amdgcn_readfirstlane(valid ? (int)rbytes : 0);
    WTile<RS> T;
    T.rsrc = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(base), (short)0, nrec, kBufferWord3);
    T.base = base;
    T.dofs = sbytes + (row * ng + kb) * 16;
    T.sofs = valid ? (row * gpr + (kb >> RS)) * 2 : 2u * (uint32_t)(kb >> RS);
    T.lastok = (ng & 3) == 0 || kb < (int)(ng & 3);
    return T;
}

template <int NS, int RS, bool SL>
__device__ __forceinline__ void down_bal_body(const GroupedArgs& a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const LayerView& L = a.L;
    const int H = L.hidden, I = L.inter, k = L.top_k;
    const int lane = lane_id(), wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int W = (int)(blockDim.x >> 6);
    constexpr int TW = kDownBalTiles;  // row tiles per unit
    const int R = (H + 16 * TW - 1) / (16 * TW);
    const Frags F = frags_at(lds, I);
    zero_block(F, threadIdx.x, blockDim.x);
    BalPlan P;
    if (!bal_plan(a, lds, I, R, R, P)) return;
    const int lo = P.lo, hi = P.hi;
    uint64_t sblob[2];
    int sp0[2], snt[2];
    const float* actp = dptr<const float>(a.W.act);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int tb = kBalToks * P.tg0[s];
        sblob[s] = P.x[s].blob;
        sp0[s] = P.x[s].p0 + tb;
        snt[s] = P.x[s].ntok - tb;
        if (s < P.nslot) {
            Frags Fs = F;
            Fs.lds = F.lds + kBalGroups * kBalPairs * s * frag_pair_bytes(F.ngp);
            const int p0 = sp0[s];
            stage_rows(Fs, P.ns[s], [&](int t) { return actp + (size_t)(p0 + t) * I; }, threadIdx.x, blockDim.x);
        }
    }
    // this wave's units: lo + wave + W * j < hi
    const int J = hi - lo > wave ? (hi - lo - wave + W - 1) / W : 0;
    const int Sx = tile_steps(I);
    const uint64_t dummy = L.router_w;
    const uint32_t swin = lds_addr_of(lds) + (uint32_t)bal_win_off(I) +
                          (uint32_t)(TW * wave * scale_window_bytes<NS>());
    auto load = [&](WRegs<NS, SL> (&B)[TW], int j, uint32_t win) {
        int s, u, gl;
        P.unit(lo + wave + W * j, s, u, gl);
        const uint64_t blob = s == 0 ? sblob[0] : sblob[1];
        const bool valid = j < J && blob != 0;
#pragma unroll
        for (int t = 0; t < TW; ++t) {
            const WTile<RS> T = wtile_dn<RS>(blob, valid, dummy, (uint32_t)L.down_off, H, I, 16 * (TW * u + t));
            wload(B[t], T, 0, win + (uint32_t)(t * scale_window_bytes<NS>()));
        }
    };
    const uint32_t y_bytes = (uint32_t)a.T * (uint32_t)k * (uint32_t)H * 4u;
    const __amdgpu_buffer_rsrc_t y_rs =
        __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(a.W.y), (short)0, (int)y_bytes, kBufferWord3);
    bool missing = false;
    auto compute = [&](const WRegs<NS, SL> (&B)[TW], int j) {
        int s, u, gl;
        P.unit(lo + wave + W * j, s, u, gl);
        const uint64_t qblob = s == 0 ? sblob[0] : sblob[1];
        const int qp0 = (s == 0 ? sp0[0] : sp0[1]) + kBalToks * gl;
        const int qnt = min(kBalToks, (s == 0 ? snt[0] : snt[1]) - kBalToks * gl);
        const int np = (qnt + 1) >> 1;
        missing |= qblob == 0;  // not resident: zero outputs, flag raised after the loop
        WRegs<NS, SL> Rm[TW];
#pragma unroll
        for (int t = 0; t < TW; ++t) {
            Rm[t] = B[t];
            if constexpr (SL) {
                // read the scale window only once the tile's first nibble load
                // has landed, and with it the window copies issued before it
                uint32_t z;
                asm("v_and_b32 %0, 0, %1" : "=v"(z) : "v"(B[t].w[0].x));
                Rm[t].sbase += z;
            }
        }
        float acc[TW][kBalPairs][2];
#pragma unroll
        for (int t = 0; t < TW; ++t)
#pragma unroll
            for (int p = 0; p < kBalPairs; ++p) acc[t][p][0] = acc[t][p][1] = 0.0f;
        ABase Bs[kBalPairs];
#pragma unroll
        for (int p = 0; p < kBalPairs; ++p) Bs[p] = abase(F, kBalPairs * (kBalGroups * s + gl) + p, 0);
        bal_wmma(Rm, Bs, Sx, np, acc);
        // the tokens' sums over K (bal_sums): one store per lane, tile and
        // group of four tokens
#pragma unroll
        for (int t = 0; t < TW; ++t) {
            float X, Y;
            bal_sums(acc[t], X, Y);
            const int row = 16 * (TW * u + t) + (lane & 15);
            const bool out = row < H;
#pragma unroll
            for (int h = 0; h < kBalPairs / 2; ++h) {
                const int tk = 4 * h + quad_row_tok(lane >> 4);
                const float v = qblob == 0 ? 0.0f : h ? Y : X;
                const bool st = out && tk < qnt;
                const uint32_t off = st ? ((uint32_t)(qp0 + tk) * (uint32_t)H + (uint32_t)row) * 4u : y_bytes;
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), y_rs, (int)off, 0, 0);
            }
        }
    };
    WRegs<NS, SL> RA[TW];
    load(RA, 0, swin);
    __builtin_amdgcn_s_waitcnt(0);  // the first unit has landed
    __syncthreads();                // and the staged act rows are in place
    for (int j = 0; j < J; ++j) {
        if (j > 0) load(RA, j, swin);
        compute(RA, j);
    }
    if (missing && lane == 0) atomicOr(gptr_w<int>(a.W.meta) + 1, kErrMissingExpert);
    __builtin_amdgcn_s_waitcnt(0);  // the last (past-the-end) unit's loads
}

// down MFMAs for one staged token group of P pairs over TW row tiles, into
// y; D holds the first chunk on entry, and ONE / reload mean what they do
// for gateup_group.
template <int P, int TW, int NS, bool ONE, int RS, bool SL>
__device__ __forceinline__ void down_group(const Frags& F, WRegs<NS, SL> (&D)[TW],
                                           const WTile<RS> (&TD)[TW], int H, const int (&n0)[TW],
                                           int S, int t0, int nt, int p0, bool reload, float* y) {
    const int np = (nt + 1) >> 1;
    const int lane = lane_id();
    float acc[TW][P][2];
#pragma unroll
    for (int tw = 0; tw < TW; ++tw)
#pragma unroll
        for (int p = 0; p < P; ++p) acc[tw][p][0] = acc[tw][p][1] = 0.0f;
    if constexpr (ONE) {
#pragma unroll
        for (int tw = 0; tw < TW; ++tw) opaque(D[tw]);
        ABase B[P];
#pragma unroll
        for (int p = 0; p < P; ++p) B[p] = abase(F, p, 0);
        wmma(D, B, S, np, acc);
    } else {
#pragma nounroll
        for (int c0 = 0;;) {
            ABase B[P];
#pragma unroll
            for (int p = 0; p < P; ++p) B[p] = abase(F, p, c0);
            wmma(D, B, S - c0, np, acc);
            c0 += NS;
            if (c0 >= S) break;
#pragma unroll
            for (int tw = 0; tw < TW; ++tw) wload(D[tw], TD[tw], c0);
        }
        if (reload) {
#pragma unroll
            for (int tw = 0; tw < TW; ++tw) wload(D[tw], TD[tw], 0);
        }
    }
#pragma unroll
    for (int tw = 0; tw < TW; ++tw) {
        const int row = n0[tw] + (lane & 15);
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const float v0 = tile_reduce(acc[tw][p][0]), v1 = tile_reduce(acc[tw][p][1]);
            const int t = 2 * p + (lane >> 4);  // within the group
            if (row < H && lane < 32 && t < nt) y[(size_t)(p0 + t0 + t) * H + row] = lane < 16 ? v0 : v1;
        }
    }
}

template <int TW, int NS, bool ONE, int RS, bool SL>
__device__ __forceinline__ void down_body(const GroupedArgs& a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const LayerView& L = a.L;
    const int H = L.hidden, I = L.inter;
    const int wave = threadIdx.x >> 6, W = blockDim.x >> 6;
    const int run = kTileRows * W * TW;
    const int chunks = (H + run - 1) / run;
    const int u = blockIdx.x / chunks;
    const int chunk = blockIdx.x - u * chunks;
    const ExpertEntry x = entry_of(a, u);
    if (x.ntok == 0) return;
    float* y = dptr<float>(a.W.y);
    if (x.blob == 0) {
        missing_expert(a, x, y, H, H, chunk * run, chunk * run + run);
        return;
    }
    const int S = tile_steps(I);
    const Frags F = frags_at(lds, I);
    WRegs<NS, SL> D[TW];
    WTile<RS> TD[TW];
    int n0[TW];
    // the wave's scale windows follow the fragment area (SL)
    const uint32_t swin = lds_addr_of(lds) + (uint32_t)frag_lds_bytes(I, a.pairs_cap) +
                          (uint32_t)(TW * wave * scale_window_bytes<NS>());
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        n0[t] = chunk * run + kTileRows * (wave + W * t);
        TD[t] = wtile<RS>(x.blob + L.down_off, H, I, n0[t]);
        wload(D[t], TD[t], 0, swin + (uint32_t)(t * scale_window_bytes<NS>()));
    }
    zero_block(F, threadIdx.x, blockDim.x);
    const float* act = dptr<const float>(a.W.act);
    const int cap = min(kMaxPairs, a.pairs_cap);
    for (int tb = 0; tb < x.ntok; tb += 2 * cap) {
        const int nt = min(2 * cap, x.ntok - tb);
        const bool reload = tb + nt < x.ntok;
        if (tb > 0) __syncthreads();
        stage_rows(F, nt, [&](int t) { return act + (size_t)(x.p0 + tb + t) * I; },
                   threadIdx.x, blockDim.x);
        __syncthreads();
        down_group<kMaxPairs, TW, NS, ONE, RS, SL>(F, D, TD, H, n0, S, tb, nt, x.p0, reload, y);
    }
}

}  // namespace

// Scale granularity (group = 32 << RS) is a template parameter so that every
// load offset of a chunk is an immediate.
#define LP_BY_RS(group, call)               \
    switch (ilog2_pow2((group) >> 5)) {      \
        case 0: call(0); break;              \
        case 1: call(1); break;              \
        default: call(2); break;             \
    }

// Gate/up: a tile of at most kGateupChunk steps is loaded in one piece and
// kept in registers; longer tiles stream kGateupLoopChunk steps at a time.
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
lp_moe_gateup(const GroupedArgs a) {
    if (tile_steps(a.L.hidden) <= kGateupChunk) {
        if (scales_in_lds(a.L.group, a.L.hidden)) {
            gateup_body<kGateupChunk, true, 0, true>(a);
        } else {
#define LP_GATEUP(rs) gateup_body<kGateupChunk, true, rs, false>(a)
            LP_BY_RS(a.L.group, LP_GATEUP)
#undef LP_GATEUP
        }
    } else {
#define LP_GATEUP(rs) gateup_body<kGateupLoopChunk, false, rs, false>(a)
        LP_BY_RS(a.L.group, LP_GATEUP)
#undef LP_GATEUP
    }
}

// Balanced gate/up (decode batches, the host checks the bounds it assumes:
// tile_steps(hidden) <= 16, at most kBalMaxU entries, no more virtual
// experts than workgroups, kBalWaves waves).
extern "C" __global__ void __launch_bounds__(64 * kBalWaves) __attribute__((amdgpu_waves_per_eu(2)))
lp_moe_gateup_bal(const GroupedArgs a) {
    gateup_bal_body<16, 0, true>(a);
}

// lp_moe_gateup_bal with the shared MLP's entries (W.sh_et, a.sh_maxu of
// them, its own width and regions, act rows into W.sh_act) planned after
// the routed ones: one launch for both.
extern "C" __global__ void __launch_bounds__(64 * kBalWaves) __attribute__((amdgpu_waves_per_eu(2)))
lp_moe_gateup_bal_sh(const GroupedArgs a) {
    gateup_bal_body<16, 0, true, true>(a);
}

// The same with tiles of at most 8 steps (hidden <= 1024), and for groups
// whose scales are not read through LDS windows (64, 128, or rows not 16-byte
// aligned).  Each form is a kernel of its own, so that each keeps its own
// register budget (together in one function they spill).
extern "C" __global__ void __launch_bounds__(64 * kBalWaves) __attribute__((amdgpu_waves_per_eu(2)))
lp_moe_gateup_bal8(const GroupedArgs a) {
    gateup_bal_body<8, 0, true>(a);
}

extern "C" __global__ void __launch_bounds__(64 * kBalWaves) __attribute__((amdgpu_waves_per_eu(2)))
lp_moe_gateup_bal_rs(const GroupedArgs a) {
#define LP_GATEUP(rs) gateup_bal_body<16, rs, false>(a)
    LP_BY_RS(a.L.group, LP_GATEUP)
#undef LP_GATEUP
}

extern "C" __global__ void __launch_bounds__(64 * kBalWaves) __attribute__((amdgpu_waves_per_eu(2)))
lp_moe_gateup_bal_rs8(const GroupedArgs a) {
#define LP_GATEUP(rs) gateup_bal_body<8, rs, false>(a)
    LP_BY_RS(a.L.group, LP_GATEUP)
#undef LP_GATEUP
}

// Balanced down (decode batches; the host checks what lp_moe_gateup_bal
// needs, with inter for hidden): units of 16 rows over all of K, tiles of 6
// steps (inter 768) or of up to 8.
extern "C" __global__ void __launch_bounds__(64 * kBalWaves) __attribute__((amdgpu_waves_per_eu(2)))
lp_moe_down_bal(const GroupedArgs a) {
    down_bal_body<8, 0, true>(a);
}

extern "C" __global__ void __launch_bounds__(64 * kBalWaves) __attribute__((amdgpu_waves_per_eu(2)))
lp_moe_down_bal6(const GroupedArgs a) {
    down_bal_body<6, 0, true>(a);
}

// Down, two row tiles per wave: tiles of at most kDownChunk steps (the host
// picks this kernel only for those), loaded in one piece.
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
lp_moe_down(const GroupedArgs a) {
    if (scales_in_lds(a.L.group, a.L.inter)) {
        // a 6-step tile (inter 768) loads only its own 6 steps
        if (tile_steps(a.L.inter) == 6)
            down_body<2, 6, true, 0, true>(a);
        else
            down_body<2, kDownChunk, true, 0, true>(a);
    } else {
#define LP_DOWN(rs) down_body<2, kDownChunk, true, rs, false>(a)
        LP_BY_RS(a.L.group, LP_DOWN)
#undef LP_DOWN
    }
}

// Down, one row tile per wave: up to kDownWideChunk steps in one piece,
// longer tiles streamed kDownLoopChunk steps at a time.
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
lp_moe_down_wide(const GroupedArgs a) {
    const int S = tile_steps(a.L.inter);
    if (S <= kDownWideChunk) {
        // tiles of 9..12 steps (inter 1152..1536) load 12 steps, not 16
        if (scales_in_lds(a.L.group, a.L.inter)) {
            if (S <= 12)
                down_body<1, 12, true, 0, true>(a);
            else
                down_body<1, kDownWideChunk, true, 0, true>(a);
        } else if (S <= 12) {
#define LP_DOWN(rs) down_body<1, 12, true, rs, false>(a)
            LP_BY_RS(a.L.group, LP_DOWN)
#undef LP_DOWN
        } else {
#define LP_DOWN(rs) down_body<1, kDownWideChunk, true, rs, false>(a)
            LP_BY_RS(a.L.group, LP_DOWN)
#undef LP_DOWN
        }
    } else {
#define LP_DOWN(rs) down_body<1, kDownLoopChunk, false, rs, false>(a)
        LP_BY_RS(a.L.group, LP_DOWN)
#undef LP_DOWN
    }
}

// ---------------------------------------------------------------------------
// Combine: h[t][i] += sum_j w[t][j] * y[inv[t*k+j]][i], j in pick order with
// fused multiply-adds, then one add (q4g64.cu:84-99); with a shared MLP its
// output is added after that, unweighted (kimi.rs:779).  Grid (ceil(H/1024),
// T): four columns per thread, eight picks' rows loaded before their FMAs;
// picks past cnt (or, for one wave of a paged union, outside it) add zeros
// with weight 0, which leaves the sum as it is.  The pick count, the first
// eight picks' rows and weights (in bounds whatever the count), the residual
// and the shared output are loaded together, so the picked rows are the only
// dependent round trip.
// ---------------------------------------------------------------------------
extern "C" __global__ void __launch_bounds__(256) lp_moe_combine(const GroupedArgs a) {
    const int t = blockIdx.y;
    const int i = (blockIdx.x * 256 + threadIdx.x) * 4;
    const int H = a.L.hidden, k = a.L.top_k;
    if (i >= H) return;
    const LP_GLOBAL int* inv = gptr<int>(a.W.inv) + (size_t)t * k;
    const LP_GLOBAL float* w = gptr<float>(a.W.wts) + (size_t)t * k;
    const LP_GLOBAL float* y = gptr<float>(a.W.y) + i;
    LP_GLOBAL float4* h = reinterpret_cast<LP_GLOBAL float4*>(gptr_w<float>(a.h) + (size_t)t * H + i);
    const int c = gptr<int>(a.W.cnt)[t];
    int iv[8];
    float wv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        iv[q] = 0;
        wv[q] = 0.0f;
        if (q < k) {
            iv[q] = inv[q];
            wv[q] = w[q];
        }
    }
    // one wave of the union (decode.rs:489-531): only picks whose dispatch
    // position lies in the wave's experts' range [p0, p1)
    int p0 = 0, p1 = 0x7fffffff;
    if (a.wave_n > 0) {
        const int u1 = min(a.wave_u0 + a.wave_n, gptr<int>(a.W.meta)[0]);
        const LP_GLOBAL int* uq = gptr<int>(a.W.uniq);
        const LP_GLOBAL int* gs = gptr<int>(a.W.gs);
        p0 = a.wave_u0 < u1 ? gs[uq[a.wave_u0]] : 0;
        p1 = a.wave_u0 < u1 ? gs[uq[u1 - 1] + 1] : 0;
    }
    float4 v = *h;
    float4 sy = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (a.L.shared_blob)
        sy = *reinterpret_cast<const LP_GLOBAL float4*>(gptr<float>(a.W.sh_y) + (size_t)t * H + i);
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    bool any = false;
    if (c > 0) {
        for (int j0 = 0; j0 < c; j0 += 8) {
            float4 yv[8];
            float wl[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int j = j0 + q;
                int r = 0;
                if (j < c) r = j0 == 0 ? iv[q] : inv[j];
                const bool live = j < c && r >= p0 && r < p1;
                any |= live;
                wl[q] = live ? (j0 == 0 ? wv[q] : w[j]) : 0.0f;
                yv[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (live) yv[q] = *reinterpret_cast<const LP_GLOBAL float4*>(y + (size_t)r * H);
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                acc.x = __builtin_fmaf(wl[q], yv[q].x, acc.x);
                acc.y = __builtin_fmaf(wl[q], yv[q].y, acc.y);
                acc.z = __builtin_fmaf(wl[q], yv[q].z, acc.z);
                acc.w = __builtin_fmaf(wl[q], yv[q].w, acc.w);
            }
        }
    }
    // a wave without any of this token's picks leaves its row as it is
    if (!any && a.wave_n > 0 && !a.L.shared_blob) return;
    if (any || a.wave_n == 0) {
        v.x = v.x + acc.x;
        v.y = v.y + acc.y;
        v.z = v.z + acc.z;
        v.w = v.w + acc.w;
    }
    if (a.L.shared_blob) {
        v.x = v.x + sy.x;
        v.y = v.y + sy.y;
        v.z = v.z + sy.z;
        v.w = v.w + sy.w;
    }
    *h = v;
}

// ---------------------------------------------------------------------------
// Down and combine of a one-token batch in one launch (lp_moe_down_comb):
// workgroup b owns rows [16 b, 16 b + 16) of h, wave w the token's pick w
// (w < cnt, at most kCombWaves picks).  Each wave stages its pick's act row
// as digit fragments in its own pair slot, loads the 16 rows of its
// expert's down matrix (one tile of at most NS steps, scales through an LDS
// window for group 32 with 16-byte aligned scale rows (SL), else read per
// lane) and leaves the 16 row sums in LDS; after a barrier the first 16
// threads fold them in pick order, h += sum_j w_j y_j, with the fused
// multiply-adds of lp_moe_combine, then add the shared MLP's row (already
// computed) as the combine does, so h is bit-identical to the down kernel
// followed by the combine.  For tile_steps(inter) <= 16 (the host checks).
//
// With sh_fused (lp_moe_down_comb_rs only; top_k <= kCombWaves -
// kCombShWaves, the shared MLP's group equal to the routed one) the last
// two waves, otherwise idle, also take the shared MLP's down for the same
// rows: its act row (already computed by the shared gate/up) staged once
// into a fragment area of its own, wave q the q-th half of its K steps,
// and the fold adds the two halves' row sums in place of the shared row.
// ---------------------------------------------------------------------------
namespace {

__host__ __device__ constexpr int comb_part_off(int inter) { return (frag_lds_bytes(inter, kCombWaves) + 15) & ~15; }

// The fused shared down's LDS (its fragment pair, then the halves' row sums)
// after the routed part's: fragments, row sums, the scale windows (SL).
__host__ __device__ constexpr int comb_sh_off(int inter, int ns, bool sl) {
    return comb_part_off(inter) + kCombWaves * 64 + (sl ? kCombWaves * 64 * 2 * ((ns + 7) / 8 * 8) : 0);
}

template <int NS, int RS, bool SL>
__device__ __forceinline__ void down_comb_body(const GroupedArgs& a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const LayerView& L = a.L;
    const int H = L.hidden, I = L.inter;
    const int lane = lane_id(), wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int n0 = kTileRows * (int)blockIdx.x;
    const int c = gptr<int>(a.W.cnt)[0];
    const Frags F = frags_at(lds, I);
    float* part = reinterpret_cast<float*>(lds + comb_part_off(I));  // [kCombWaves][16]
    const uint32_t swin = lds_addr_of(lds) + (uint32_t)(comb_part_off(I) + kCombWaves * 64) +
                          (uint32_t)(wave * scale_window_bytes<NS>());
    zero_block(F, threadIdx.x, blockDim.x);
    // the pick's dispatch position; with one token, entry p of the expert
    // table holds position p alone.  Read without waiting for the count
    // (clamped into the table: positions of dropped picks are stale).
    const int p = min(max(gptr<int>(a.W.inv)[min(wave, L.top_k - 1)], 0), a.maxu - 1);
    const uint64_t eb = entry_of(a, p).blob;
    const uint64_t blob = wave < c ? eb : 0;
    // the fused shared down (sh_fused, per-lane scales only): wave q of the
    // last kCombShWaves takes steps [q hs, q hs + hs) of its tile
    constexpr bool kSh = !SL && NS == 16;
    const bool fused = kSh && a.sh_fused != 0;
    const bool shw = fused && wave >= kCombWaves - kCombShWaves;
    const int q = wave - (kCombWaves - kCombShWaves);
    const int Is = fused ? L.shared_inter : 32;
    const int Ss = tile_steps(Is), hs = (Ss + kCombShWaves - 1) / kCombShWaves;
    uint8_t* sh_lds = lds + comb_sh_off(I, NS, SL);
    const Frags Fs = frags_at(sh_lds, Is);
    float* psh = reinterpret_cast<float*>(sh_lds + ((frag_lds_bytes(Is, 1) + 15) & ~15));  // [kCombShWaves][16]
    if (fused) zero_block(Fs, threadIdx.x, blockDim.x);
    WRegs<NS, SL> D;
    if (blob != 0) {
        const WTile<RS> T = wtile<RS>(blob + L.down_off, H, I, n0);
        wload(D, T, 0, swin);
        Frags Fw = F;
        Fw.lds = F.lds + wave * frag_pair_bytes(F.ngp);
        const float* actp = dptr<const float>(a.W.act);
        stage_rows(Fw, 1, [&](int) { return actp + (size_t)p * I; }, lane, 64);
    } else if (shw) {
        const WTile<RS> T = wtile<RS>(L.shared_blob + L.sh_down_off, H, Is, n0);
        wload(D, T, q * hs, swin);
        const float* sact = dptr<const float>(a.W.sh_act);
        stage_rows(Fs, 1, [&](int) { return sact; }, (int)threadIdx.x - 64 * (kCombWaves - kCombShWaves),
                   64 * kCombShWaves);
    }
    __builtin_amdgcn_s_waitcnt(0);  // the tile, its scale window and the staged row
    __syncthreads();
    float yv = 0.0f;
    if (blob != 0) {
        float acc[1][1][2] = {{{0.0f, 0.0f}}};
        const ABase B[1] = {abase(F, wave, 0)};
        const WRegs<NS, SL> Rm[1] = {D};
        wmma(Rm, B, tile_steps(I), 1, acc);
        yv = tile_reduce(acc[0][0][0]);
    } else if (wave < c && lane == 0) {
        atomicOr(gptr_w<int>(a.W.meta) + 1, kErrMissingExpert);  // not resident: zero output
    } else if (shw) {
        // this half's steps only: the first half never reaches the tile's
        // last step, whose lanes past the last sub-group take a zero scale
        float acc[1][1][2] = {{{0.0f, 0.0f}}};
        const ABase B[1] = {abase(Fs, 0, q * hs)};
        WRegs<NS, SL> Rm[1] = {D};
        if (q + 1 < kCombShWaves) Rm[0].lastok = true;
        wmma(Rm, B, min(hs, Ss - q * hs), 1, acc);
        const float ys = tile_reduce(acc[0][0][0]);
        if (lane < 16) psh[q * 16 + lane] = ys;
    }
    if (lane < 16) part[wave * 16 + lane] = yv;
    __syncthreads();
    const int row = n0 + (int)threadIdx.x;
    if (threadIdx.x < 16 && row < H) {
        const LP_GLOBAL float* w = gptr<float>(a.W.wts);
        float acc = 0.0f;
        for (int j = 0; j < c; ++j) acc = __builtin_fmaf(w[j], part[j * 16 + threadIdx.x], acc);
        LP_GLOBAL float* h = gptr_w<float>(a.h);
        float v = h[row] + acc;
        if (L.shared_blob) {
            float sy;
            if (fused)
                sy = psh[threadIdx.x] + psh[16 + threadIdx.x];
            else
                sy = gptr<float>(a.W.sh_y)[row];
            v = v + sy;
        }
        h[row] = v;
    }
}

}  // namespace

extern "C" __global__ void __launch_bounds__(64 * kCombWaves) lp_moe_down_comb(const GroupedArgs a) {
    if (tile_steps(a.L.inter) == 6)
        down_comb_body<6, 0, true>(a);  // inter 768 loads only its own 6 steps
    else
        down_comb_body<8, 0, true>(a);
}

extern "C" __global__ void __launch_bounds__(64 * kCombWaves) lp_moe_down_comb16(const GroupedArgs a) {
    down_comb_body<16, 0, true>(a);
}

// Scales read per lane (groups 64 and 128, or scale rows not 16-byte aligned).
extern "C" __global__ void __launch_bounds__(64 * kCombWaves) lp_moe_down_comb_rs(const GroupedArgs a) {
#define LP_DOWN(rs) down_comb_body<16, rs, false>(a)
    LP_BY_RS(a.L.group, LP_DOWN)
#undef LP_DOWN
}
