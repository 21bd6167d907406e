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

// IEEE binary32 division, correctly rounded: the binary64 quotient of two
// binary32 values rounds to the same binary32 as the exact quotient (53 >= 2*24+2).
__device__ __forceinline__ float div_rn(float a, float b) { return (float)((double)a / (double)b); }

}  // namespace

// ---------------------------------------------------------------------------
// Router GEMV: logits[t][e] = W_r[e, :] . x[t, :] (bf16 x f32, fp32 FMAs) in the
// canonical order: lane l takes 8-column chunks l, l+64, ... with fused
// multiply-adds, then a butterfly over the 64 lanes.  One wave per expert row,
// kRouterTokBlock tokens per wave.  Grid (ceil(E/4), ceil(T/8)).
// ---------------------------------------------------------------------------
extern "C" __global__ void __launch_bounds__(256) lp_moe_router(const RouteArgs a) {
    const int wave = threadIdx.x >> 6;
    const int lane = lane_id();
    const int E = a.L.experts, H = a.L.hidden;
    const int e = blockIdx.x * 4 + wave;
    const int t0 = blockIdx.y * kRouterTokBlock;
    if (e >= E) return;
    const int nt = min(kRouterTokBlock, a.T - t0);
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
        if (lane == 0 && t < nt) logits[(size_t)(t0 + t) * E + e] = v;
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
extern "C" __global__ void __launch_bounds__(256) lp_moe_topk(const RouteArgs a) {
    __shared__ float sh_v[4][kMaxExperts];
    const int wave = threadIdx.x >> 6;
    const int lane = lane_id();
    const int t = blockIdx.x * 4 + wave;
    if (t >= a.T) return;
    const int E = a.L.experts, k = a.L.top_k;
    constexpr int PER = kMaxExperts / 64;
    const float* lg = dptr<const float>(a.W.logits) + (size_t)t * E;
    float* sv = sh_v[wave];
    uint32_t key[PER];

    if (a.L.gating == 0) {
        float m = -3.40282347e+38f;  // f32::MIN
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = lane + 64 * q;
            if (i < E) m = fmaxf(m, lg[i]);
        }
        m = wave_max(m);
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = lane + 64 * q;
            if (i < E) sv[i] = expf_glibc(lg[i] - m);
        }
        wave_sync_lds();
        float z = 0.0f;
        if (lane == 0) {
            z = -0.0f;
            for (int i = 0; i < E; ++i) z = z + sv[i];
        }
        z = __shfl(z, 0, 64);
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = lane + 64 * q;
            key[q] = 0u;
            if (i < E) {
                const float p = div_rn(sv[i], z);
                key[q] = ordered_key(p);
            }
        }
        wave_sync_lds();
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = lane + 64 * q;
            if (i < E) sv[i] = div_rn(sv[i], z);
        }
    } else {
        const float* bias = dptr<const float>(a.L.router_bias);
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = lane + 64 * q;
            key[q] = 0u;
            if (i < E) {
                const float d = 1.0f + expf_glibc(-lg[i]);
                const float s = div_rn(1.0f, d);
                sv[i] = s;
                key[q] = ordered_key((s + bias[i]) + 0.0f);  // -0 ranks equal to +0
            }
        }
    }
    wave_sync_lds();

    const int n = k < E ? k : E;
    uint32_t picked = 0u;
    int ids[kMaxTopK];
    float val[kMaxTopK];
    for (int j = 0; j < n; ++j) {
        uint64_t best = 0;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = lane + 64 * q;
            if (i < E && !((picked >> q) & 1u)) {
                const uint64_t c = ((uint64_t)key[q] << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
                best = c > best ? c : best;
            }
        }
        best = wave_max_u64(best);
        const int id = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
        if ((id & 63) == lane) picked |= 1u << (id >> 6);
        ids[j] = id;
        val[j] = sv[id];
    }

    int kept = n;
    float w[kMaxTopK];
    float s = -0.0f;
    for (int j = 0; j < n; ++j) s = s + val[j];
    if (a.L.gating == 0) {
        for (int j = 0; j < n; ++j) w[j] = a.L.renorm ? div_rn(val[j], s) : val[j];
    } else {
        for (int j = 0; j < n; ++j) {
            float v = val[j];
            if (a.L.renorm && s > 0.0f) v = div_rn(v, s);
            w[j] = v * a.L.routed_scaling;
        }
        if (a.L.min_weight > 0.0f) {
            kept = 0;
            for (int j = 0; j < n; ++j) {
                if (w[j] >= a.L.min_weight) {
                    ids[kept] = ids[j];
                    w[kept] = w[j];
                    ++kept;
                }
            }
        }
    }
    if (lane == 0) {
        int* gids = dptr<int>(a.W.ids) + (size_t)t * k;
        float* gw = dptr<float>(a.W.wts) + (size_t)t * k;
        for (int j = 0; j < k; ++j) {
            gids[j] = j < kept ? ids[j] : -1;
            gw[j] = j < kept ? w[j] : 0.0f;
        }
        dptr<int>(a.W.cnt)[t] = kept;
    }
}

// ---------------------------------------------------------------------------
// Dispatch (one wave): the (t, j) picks stably grouped by expert id, then t
// ascending.  Writes group starts gs[E+1], perm[pos] = t*k + j, inv[t*k + j] =
// pos (-1 for unused pick slots), uniq[] (experts with picks, ascending) and
// meta[0] = unique count; clears meta[1] (error flags).  Stability comes from
// ranking each pick by the tokens before it inside a 64-token block (one bit
// per lane) plus a running per-expert base across blocks.
// ---------------------------------------------------------------------------
extern "C" __global__ void __launch_bounds__(64) lp_moe_dispatch(const RouteArgs a) {
    __shared__ int cnt_e[kMaxExperts];
    __shared__ int base[kMaxExperts];
    __shared__ int gsl[kMaxExperts + 1];
    __shared__ uint32_t mlo[kMaxExperts];
    __shared__ uint32_t mhi[kMaxExperts];
    const int lane = lane_id();
    const int E = a.L.experts, k = a.L.top_k, T = a.T;
    const int* ids = dptr<const int>(a.W.ids);
    const int* cnt = dptr<const int>(a.W.cnt);
    int* perm = dptr<int>(a.W.perm);
    int* inv = dptr<int>(a.W.inv);
    int* meta = dptr<int>(a.W.meta);

    for (int e = lane; e < E; e += 64) {
        cnt_e[e] = 0;
        base[e] = 0;
    }
    __syncthreads();
    for (int p = lane; p < T * k; p += 64) {
        const int t = p / k, j = p - t * k;
        if (j < cnt[t]) atomicAdd(&cnt_e[ids[p]], 1);
    }
    __syncthreads();
    if (lane == 0) {
        int* uniq = dptr<int>(a.W.uniq);
        int nu = 0;
        gsl[0] = 0;
        for (int e = 0; e < E; ++e) {
            gsl[e + 1] = gsl[e] + cnt_e[e];
            if (cnt_e[e] > 0) uniq[nu++] = e;
        }
        meta[0] = nu;
        meta[1] = 0;
    }
    __syncthreads();
    int* gs = dptr<int>(a.W.gs);
    for (int e = lane; e <= E; e += 64) gs[e] = gsl[e];

    for (int tb = 0; tb < T; tb += 64) {
        for (int e = lane; e < E; e += 64) {
            mlo[e] = 0u;
            mhi[e] = 0u;
        }
        __syncthreads();
        const int t = tb + lane;
        const int c = t < T ? cnt[t] : 0;
        for (int j = 0; j < c; ++j) {
            const int e = ids[t * k + j];
            atomicOr(lane < 32 ? &mlo[e] : &mhi[e], 1u << (lane & 31));
        }
        __syncthreads();
        if (t < T) {
            for (int j = 0; j < k; ++j) {
                if (j < c) {
                    const int e = ids[t * k + j];
                    const uint64_t mask = (uint64_t)mlo[e] | ((uint64_t)mhi[e] << 32);
                    const uint64_t below = lane == 0 ? 0ull : (mask & ((1ull << lane) - 1ull));
                    const int pos = gsl[e] + base[e] + __popcll(below);
                    perm[pos] = t * k + j;
                    inv[t * k + j] = pos;
                } else {
                    inv[t * k + j] = -1;
                }
            }
        }
        __syncthreads();
        for (int e = lane; e < E; e += 64) base[e] += __popc(mlo[e]) + __popc(mhi[e]);
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Grouped expert projections.  A workgroup of W waves takes one work item =
// (unique expert, run of rows); every wave owns 16-row tiles of that run and
// the workgroup stages the expert's tokens into shared LDS fragments, up to
// `pairs_cap` token pairs at a time.  Weight loads are issued before the
// fragments are staged, and each dequantised weight word serves every staged
// token pair.
//   gate/up: act[pos][r] = silu(gate_e . x_t)[r] * (up_e . x_t)[r], r < I
//   down:    y[pos][r]   = (down_e . act[pos])[r], r < H
// pos = dispatch position of the (token, pick) pair; expert e's blob sits at
// arena_base + slot_table[e] * slot_span (the per-layer slot arena of
// pager.rs:310-318).  An expert without a slot raises kErrMissingExpert in
// meta[1] and its outputs are zero.
// ---------------------------------------------------------------------------
namespace {

struct Item {
    int e, slot, p0, ntok, chunk;
    bool live;
};

__device__ __forceinline__ Item item_of(const GroupedArgs& a, int chunks) {
    Item it;
    const int nu = gptr<int>(a.W.meta)[0];
    const int u = blockIdx.x / chunks;
    it.live = u < nu;
    if (!it.live) return it;
    it.chunk = blockIdx.x - u * chunks;
    it.e = gptr<int>(a.W.uniq)[u];
    it.slot = gptr<int>(a.L.slot_table)[it.e];
    it.p0 = gptr<int>(a.W.gs)[it.e];
    it.ntok = gptr<int>(a.W.gs)[it.e + 1] - it.p0;
    return it;
}

__device__ __forceinline__ void missing_expert(const GroupedArgs& a, const Item& it, float* out,
                                               int stride, int rows, int row_lo, int row_hi) {
    if (threadIdx.x == 0) atomicOr(dptr<int>(a.W.meta) + 1, kErrMissingExpert);
    for (int p = 0; p < it.ntok; ++p)
        for (int r = row_lo + (int)threadIdx.x; r < row_hi && r < rows; r += blockDim.x)
            out[(size_t)(it.p0 + p) * stride + r] = 0.0f;
}

template <int NS, int PMAX>
__device__ __forceinline__ void gateup_body(const GroupedArgs& a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const LayerView& L = a.L;
    const int H = L.hidden, I = L.inter, k = L.top_k;
    const int wave = threadIdx.x >> 6, W = blockDim.x >> 6, lane = lane_id();
    const int ng = H >> 5;
    const int run = kTileRows * W;
    const int chunks = (I + run - 1) / run;
    const Item it = item_of(a, chunks);
    if (!it.live) return;
    float* act = dptr<float>(a.W.act);
    if (it.slot < 0) {
        missing_expert(a, it, act, I, I, it.chunk * run, it.chunk * run + run);
        return;
    }
    const uint64_t blob = L.arena_base + (uint64_t)it.slot * L.slot_span;
    const uint64_t rg = blob + L.gate_off, ru = blob + L.up_off;
    const int rs = ilog2_pow2(L.group >> 5);
    const int S = tile_steps(H);
    const int n0 = it.chunk * run + kTileRows * wave;
    const int row = n0 + (lane & 15);
    const int cap = min(PMAX, a.pairs_cap);
    const Frags F = frags_at(lds, ng, cap);
    const bool one = S <= NS;
    WRegs<NS> G, U;
    if (one) {
        wload(G, rg, I, H, rs, n0, 0);
        wload(U, ru, I, H, rs, n0, 0);
    }
    const int* perm = dptr<const int>(a.W.perm);
    const float* x = dptr<const float>(a.x);
    for (int tb = 0; tb < it.ntok; tb += 2 * cap) {
        const int nt = min(2 * cap, it.ntok - tb);
        const int pairs = (nt + 1) >> 1;
        if (tb > 0) __syncthreads();
        stage_rows(F, nt, [&](int t) { return x + (size_t)(perm[it.p0 + tb + t] / k) * H; },
                   threadIdx.x, blockDim.x);
        __syncthreads();
        float ag[PMAX][2], au[PMAX][2];
#pragma unroll
        for (int p = 0; p < PMAX; ++p) ag[p][0] = ag[p][1] = au[p][0] = au[p][1] = 0.0f;
        for (int c0 = 0; c0 < S; c0 += NS) {
            if (!one) {
                wload(G, rg, I, H, rs, n0, c0);
                wload(U, ru, I, H, rs, n0, c0);
            }
            wmma(G, F, H, c0, pairs, ag);
            wmma(U, F, H, c0, pairs, au);
        }
#pragma unroll
        for (int p = 0; p < PMAX; ++p) {
            if (p < pairs) {
                const float g0 = tile_reduce(ag[p][0]), g1 = tile_reduce(ag[p][1]);
                const float u0 = tile_reduce(au[p][0]), u1 = tile_reduce(au[p][1]);
                const int t = tb + 2 * p + (lane >> 4);
                if (row < I && lane < 32 && t < it.ntok) {
                    const float g = lane < 16 ? g0 : g1;
                    const float u = lane < 16 ? u0 : u1;
                    act[(size_t)(it.p0 + t) * I + row] = g / (1.0f + expf(-g)) * u;
                }
            }
        }
    }
}

template <int NS, int TW, int PMAX>
__device__ __forceinline__ void down_body(const GroupedArgs& a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const LayerView& L = a.L;
    const int H = L.hidden, I = L.inter;
    const int wave = threadIdx.x >> 6, W = blockDim.x >> 6, lane = lane_id();
    const int ng = I >> 5;
    const int run = kTileRows * W * TW;
    const int chunks = (H + run - 1) / run;
    const Item it = item_of(a, chunks);
    if (!it.live) return;
    float* y = dptr<float>(a.W.y);
    if (it.slot < 0) {
        missing_expert(a, it, y, H, H, it.chunk * run, it.chunk * run + run);
        return;
    }
    const uint64_t rd = L.arena_base + (uint64_t)it.slot * L.slot_span + L.down_off;
    const int rs = ilog2_pow2(L.group >> 5);
    const int S = tile_steps(I);
    const int cap = min(PMAX, a.pairs_cap);
    const Frags F = frags_at(lds, ng, cap);
    const bool one = S <= NS;
    WRegs<NS> D[TW];
    int n0[TW];
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        n0[t] = it.chunk * run + kTileRows * (wave + W * t);
        if (one) wload(D[t], rd, H, I, rs, n0[t], 0);
    }
    const float* act = dptr<const float>(a.W.act);
    for (int tb = 0; tb < it.ntok; tb += 2 * cap) {
        const int nt = min(2 * cap, it.ntok - tb);
        const int pairs = (nt + 1) >> 1;
        if (tb > 0) __syncthreads();
        stage_rows(F, nt, [&](int t) { return act + (size_t)(it.p0 + tb + t) * I; },
                   threadIdx.x, blockDim.x);
        __syncthreads();
#pragma unroll
        for (int tw = 0; tw < TW; ++tw) {
            float acc[PMAX][2];
#pragma unroll
            for (int p = 0; p < PMAX; ++p) acc[p][0] = acc[p][1] = 0.0f;
            for (int c0 = 0; c0 < S; c0 += NS) {
                if (!one) wload(D[tw], rd, H, I, rs, n0[tw], c0);
                wmma(D[tw], F, I, c0, pairs, acc);
            }
            const int row = n0[tw] + (lane & 15);
#pragma unroll
            for (int p = 0; p < PMAX; ++p) {
                if (p < pairs) {
                    const float v0 = tile_reduce(acc[p][0]), v1 = tile_reduce(acc[p][1]);
                    const int t = tb + 2 * p + (lane >> 4);
                    if (row < H && lane < 32 && t < it.ntok)
                        y[(size_t)(it.p0 + t) * H + row] = lane < 16 ? v0 : v1;
                }
            }
        }
    }
}

}  // namespace

extern "C" __global__ void __launch_bounds__(256) lp_moe_gateup(const GroupedArgs a) {
    gateup_body<16, kMaxPairs>(a);
}

extern "C" __global__ void __launch_bounds__(256) lp_moe_down(const GroupedArgs a) {
    down_body<8, 2, kMaxPairs>(a);
}

extern "C" __global__ void __launch_bounds__(256) lp_moe_down_wide(const GroupedArgs a) {
    down_body<16, 1, kMaxPairs>(a);
}

// ---------------------------------------------------------------------------
// Combine: h[t][i] += sum_j w[t][j] * y[inv[t*k+j]][i], j in pick order with
// fused multiply-adds, then one add (q4g64.cu:84-99).  Grid (ceil(H/256), T).
// ---------------------------------------------------------------------------
extern "C" __global__ void __launch_bounds__(256) lp_moe_combine(const GroupedArgs a) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int H = a.L.hidden, k = a.L.top_k;
    if (i >= H) return;
    const int c = dptr<const int>(a.W.cnt)[t];
    const int* inv = dptr<const int>(a.W.inv) + (size_t)t * k;
    const float* w = dptr<const float>(a.W.wts) + (size_t)t * k;
    const float* y = dptr<const float>(a.W.y);
    float acc = 0.0f;
    for (int j = 0; j < c; ++j) acc = __builtin_fmaf(w[j], y[(size_t)inv[j] * H + i], acc);
    float* h = dptr<float>(a.h) + (size_t)t * H;
    h[i] += acc;
}
