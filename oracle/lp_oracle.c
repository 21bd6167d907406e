/*
 * lp_oracle.c -- CPU restatement of llmpager's MoE-layer hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see lp_oracle.h).  Built with -ffp-contract=off
 * so that every a*b+c below rounds twice, as rustc's output does; the two
 * places that fuse on purpose call fmaf() explicitly and say why.
 */
#include "lp_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---- conversions -------------------------------------------------------- */

/* quant.rs:151-171 */
uint16_t lpo_f32_to_f16_ref(float x) {
    uint32_t b = f2u(x);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    int32_t exp = (int32_t)((b >> 23) & 0xFFu);
    uint32_t frac = b & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (frac != 0 ? 0x200u : 0u));
    int32_t e = exp - 127 + 15;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = (frac | 0x800000u) >> (1 - e);
        return (uint16_t)(sign | (uint16_t)((m + 0x1000u) >> 13));
    }
    /* The rounding carry is OR-ed into the exponent field (quant.rs:170). */
    return (uint16_t)(sign | (uint16_t)((uint32_t)e << 10) | (uint16_t)((frac + 0x1000u) >> 13));
}

/* quant.rs:173-189 */
float lpo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)(h & 0x8000u)) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t frac = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0 && frac == 0) {
        bits = sign;
    } else if (exp == 0) {
        uint32_t shift = (uint32_t)__builtin_clz(frac) - 21;
        bits = sign | ((127 - 15 - shift + 1) << 23) | ((frac << (shift + 13)) & 0x7FFFFFu);
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (frac << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (frac << 13);
    }
    return u2f(bits);
}

/* kernels_bench.rs:20-22, decode.cu:8-11 */
float lpo_bf16_to_f32(uint16_t h) { return u2f(((uint32_t)h) << 16); }

float lpo_expf(float x) { return expf(x); }

void lpo_expf_sweep(uint32_t first, uint32_t stride, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = expf(u2f(first + (uint32_t)(i * stride)));
}

/* Rust's f32 `Iterator::sum` folds from -0.0 (rustc >= 1.81); starting there
 * only changes the sign of an all-zero sum. */
#define RUST_SUM_INIT (-0.0f)

/* ---- q4 format ---------------------------------------------------------- */

size_t lpo_q4_bytes(size_t rows, size_t cols, size_t group) {
    return rows * (cols / group) * 2 + rows * cols / 2;
}

static float f16_round_ref(float x) { return lpo_f16_to_f32(lpo_f32_to_f16_ref(x)); }

/* quant.rs:102-109 */
static int32_t quantize_one(float x, float scale, float* max_err) {
    float q = roundf(x / scale);
    if (q < -8.0f) q = -8.0f;
    if (q > 7.0f) q = 7.0f;
    int32_t qi = (int32_t)q;
    float err = fabsf(x - (float)qi * scale);
    if (err > *max_err) *max_err = err;
    return qi + 8;
}

/* quant.rs:37-76 */
int lpo_q4_quantize(const float* src, size_t rows, size_t cols, size_t group,
                    uint8_t* dst, size_t dst_len, float* max_err_out) {
    if (group == 0 || group % 8 != 0 || cols % group != 0) return -1;
    if (dst_len != lpo_q4_bytes(rows, cols, group)) return -1;
    size_t gpr = cols / group;
    uint8_t* scales = dst;
    uint8_t* data = dst + rows * gpr * 2;
    float max_err = 0.0f;
    for (size_t r = 0; r < rows; ++r) {
        for (size_t g = 0; g < gpr; ++g) {
            const float* vals = src + r * cols + g * group;
            float amax = 0.0f;
            for (size_t i = 0; i < group; ++i) amax = fmaxf(amax, fabsf(vals[i]));
            float scale = fmaxf(f16_round_ref(amax > 0.0f ? amax / 7.0f : 1e-8f), 1e-7f);
            uint16_t sb = lpo_f32_to_f16_ref(scale);
            size_t sidx = (r * gpr + g) * 2;
            scales[sidx] = (uint8_t)(sb & 0xFF);
            scales[sidx + 1] = (uint8_t)(sb >> 8);
            size_t base = r * cols / 2 + g * group / 2;
            for (size_t i = 0; i < group / 2; ++i) {
                int32_t q0 = quantize_one(vals[2 * i], scale, &max_err);
                int32_t q1 = quantize_one(vals[2 * i + 1], scale, &max_err);
                data[base + i] = (uint8_t)(((uint8_t)q0 & 0x0F) | (((uint8_t)q1 & 0x0F) << 4));
            }
        }
    }
    if (max_err_out) *max_err_out = max_err;
    return 0;
}

/* quant.rs:81-100 */
void lpo_q4_store_group(uint8_t* dst, size_t rows, size_t cols, size_t group,
                        size_t row, size_t g, float scale, const uint8_t* qs) {
    size_t gpr = cols / group;
    uint8_t* data = dst + rows * gpr * 2;
    uint16_t sb = lpo_f32_to_f16_ref(scale);
    size_t sidx = (row * gpr + g) * 2;
    dst[sidx] = (uint8_t)(sb & 0xFF);
    dst[sidx + 1] = (uint8_t)(sb >> 8);
    size_t base = row * cols / 2 + g * group / 2;
    for (size_t i = 0; i < group / 2; ++i)
        data[base + i] = (uint8_t)((qs[2 * i] & 0x0F) | ((qs[2 * i + 1] & 0x0F) << 4));
}

/* quant.rs:117-147 */
int lpo_q4_dequantize(const uint8_t* buf, size_t buf_len, size_t rows,
                      size_t cols, size_t group, float* out) {
    if (group == 0 || cols % group != 0 || buf_len != lpo_q4_bytes(rows, cols, group)) return -1;
    size_t gpr = cols / group;
    const uint8_t* data = buf + rows * gpr * 2;
    for (size_t r = 0; r < rows; ++r) {
        for (size_t g = 0; g < gpr; ++g) {
            size_t sidx = (r * gpr + g) * 2;
            float scale = lpo_f16_to_f32((uint16_t)(buf[sidx] | (buf[sidx + 1] << 8)));
            size_t base = r * cols / 2 + g * group / 2;
            for (size_t i = 0; i < group / 2; ++i) {
                uint8_t b = data[base + i];
                out[r * cols + g * group + 2 * i] = (float)((int32_t)(b & 0x0F) - 8) * scale;
                out[r * cols + g * group + 2 * i + 1] = (float)((int32_t)(b >> 4) - 8) * scale;
            }
        }
    }
    return 0;
}

/* ---- kernel CPU forms ----------------------------------------------------- */

/* One output row of the gemv_bench.rs:30-41 form: the value dequantised as in
 * quant.rs:141-142 (exact in f32), times x, summed sequentially. */
static float q4_row(const uint8_t* region, const float* x, int rows, int cols,
                    int group, int r) {
    int gpr = cols / group;
    const uint8_t* scales = region + (size_t)r * gpr * 2;
    const uint8_t* data = region + (size_t)rows * gpr * 2 + (size_t)r * (cols / 2);
    float acc = RUST_SUM_INIT;
    for (int g = 0; g < gpr; ++g) {
        float s = lpo_f16_to_f32((uint16_t)(scales[2 * g] | (scales[2 * g + 1] << 8)));
        const uint8_t* d = data + (size_t)g * (group / 2);
        const float* xg = x + (size_t)g * group;
        for (int i = 0; i < group / 2; ++i) {
            uint8_t b = d[i];
            float w0 = (float)((int32_t)(b & 0x0F) - 8) * s;
            float w1 = (float)((int32_t)(b >> 4) - 8) * s;
            acc = acc + w0 * xg[2 * i];
            acc = acc + w1 * xg[2 * i + 1];
        }
    }
    return acc;
}

static void q4_gemv_mt(const uint8_t* region, const float* x, float* y, int rows,
                       int cols, int group, int threads) {
#ifdef _OPENMP
    if (threads > 1) {
#pragma omp parallel for num_threads(threads) schedule(static)
        for (int r = 0; r < rows; ++r) y[r] = q4_row(region, x, rows, cols, group, r);
        return;
    }
#endif
    (void)threads;
    for (int r = 0; r < rows; ++r) y[r] = q4_row(region, x, rows, cols, group, r);
}

void lpo_q4_gemv(const uint8_t* region, const float* x, float* y, int rows,
                 int cols, int group) {
    q4_gemv_mt(region, x, y, rows, cols, group, 1);
}

void lpo_q4_gemv_batch(const uint8_t* const* blobs, uint64_t region_off,
                       const float* x, int x_stride, float* y, int rows,
                       int cols, int group, int experts) {
    for (int e = 0; e < experts; ++e)
        lpo_q4_gemv(blobs[e] + region_off, x + (size_t)e * x_stride, y + (size_t)e * rows,
                    rows, cols, group);
}

void lpo_bf16_gemv(const uint16_t* w, const float* x, float* y, int rows, int cols) {
    for (int r = 0; r < rows; ++r) {
        float acc = RUST_SUM_INIT;
        for (int c = 0; c < cols; ++c) acc = acc + lpo_bf16_to_f32(w[(size_t)r * cols + c]) * x[c];
        y[r] = acc;
    }
}

void lpo_silu_mul(const float* gate, const float* up, float* out, int n) {
    for (int i = 0; i < n; ++i) {
        float g = gate[i];
        out[i] = g / (1.0f + expf(-g)) * up[i];
    }
}

/* q4g64.cu:84-99.  nvcc contracts `a += wts[e] * eouts[..]` into an FMA
 * (its default), so the restatement fuses too. */
void lpo_moe_reduce(const float* eouts, const float* wts, float* out, int experts, int n) {
    for (int i = 0; i < n; ++i) {
        float a = 0.0f;
        for (int e = 0; e < experts; ++e) a = fmaf(wts[e], eouts[(size_t)e * n + i], a);
        out[i] += a;
    }
}

void lpo_add(float* a, const float* b, int n) {
    for (int i = 0; i < n; ++i) a[i] += b[i];
}

/* ---- routing ---------------------------------------------------------- */

/* Stable sort of idx[0..n) by key descending; equal keys (== in IEEE terms,
 * so -0 == +0) keep their order, as slice::sort_by with partial_cmp does. */
static void stable_sort_desc(int32_t* idx, const float* key, int n) {
    for (int i = 1; i < n; ++i) {
        int32_t v = idx[i];
        float kv = key[v];
        int j = i;
        while (j > 0 && key[idx[j - 1]] < kv) {
            idx[j] = idx[j - 1];
            --j;
        }
        idx[j] = v;
    }
}

/* decode.rs:734-749 */
int lpo_top_k_softmax(const float* logits, int E, int k, int renorm, int32_t* ids, float* w) {
    if (E <= 0 || k <= 0) return 0;
    float m = -3.40282347e+38f; /* f32::MIN */
    for (int i = 0; i < E; ++i) m = fmaxf(m, logits[i]);
    float* p = (float*)malloc(sizeof(float) * (size_t)E);
    int32_t* idx = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    float z = RUST_SUM_INIT;
    for (int i = 0; i < E; ++i) {
        p[i] = expf(logits[i] - m);
        z = z + p[i];
    }
    for (int i = 0; i < E; ++i) {
        p[i] = p[i] / z;
        idx[i] = i;
    }
    stable_sort_desc(idx, p, E);
    int n = k < E ? k : E;
    float s = RUST_SUM_INIT;
    for (int j = 0; j < n; ++j) {
        ids[j] = idx[j];
        w[j] = p[idx[j]];
        s = s + w[j];
    }
    if (renorm)
        for (int j = 0; j < n; ++j) w[j] = w[j] / s;
    free(p);
    free(idx);
    return n;
}

/* kimi.rs:1155-1186 */
int lpo_sigmoid_topk(const float* logits, const float* bias, int E, int k, int renorm,
                     float scaling, float min_weight, int32_t* ids, float* w) {
    if (E <= 0 || k <= 0) return 0;
    float* sc = (float*)malloc(sizeof(float) * (size_t)E);
    float* key = (float*)malloc(sizeof(float) * (size_t)E);
    int32_t* idx = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    for (int i = 0; i < E; ++i) {
        sc[i] = 1.0f / (1.0f + expf(-logits[i]));
        key[i] = sc[i] + bias[i];
        idx[i] = i;
    }
    stable_sort_desc(idx, key, E);
    int n = k < E ? k : E;
    float s = RUST_SUM_INIT;
    for (int j = 0; j < n; ++j) {
        ids[j] = idx[j];
        w[j] = sc[idx[j]];
        s = s + w[j];
    }
    if (renorm && s > 0.0f)
        for (int j = 0; j < n; ++j) w[j] = w[j] / s;
    for (int j = 0; j < n; ++j) w[j] = w[j] * scaling;
    int kept = n;
    if (min_weight > 0.0f) {
        kept = 0;
        for (int j = 0; j < n; ++j) {
            if (w[j] >= min_weight) {
                ids[kept] = ids[j];
                w[kept] = w[j];
                ++kept;
            }
        }
    }
    free(sc);
    free(key);
    free(idx);
    return kept;
}

void lpo_router_logits(const uint16_t* w, const float* x, float* logits, int E, int H) {
    int chunks = H / 8;
    for (int e = 0; e < E; ++e) {
        const uint16_t* row = w + (size_t)e * H;
        float lane[64], tmp[64];
        for (int l = 0; l < 64; ++l) {
            float acc = 0.0f;
            for (int ch = l; ch < chunks; ch += 64)
                for (int i = 0; i < 8; ++i) {
                    int c = ch * 8 + i;
                    /* the HIP kernel issues v_fma_f32 here, so this fuses on purpose */
                    acc = fmaf(lpo_bf16_to_f32(row[c]), x[c], acc);
                }
            lane[l] = acc;
        }
        for (int off = 32; off >= 1; off >>= 1) {
            for (int l = 0; l < 64; ++l) tmp[l] = lane[l] + lane[l ^ off];
            memcpy(lane, tmp, sizeof(lane));
        }
        logits[e] = lane[0];
    }
}

/* ---- dispatch ------------------------------------------------------------ */

int lpo_moe_dispatch(const int32_t* ids, const int32_t* cnt, int T, int k, int E,
                     int32_t* perm, int32_t* group_start, int32_t* inv, int32_t* uniq) {
    int32_t* count = (int32_t*)calloc((size_t)E + 1, sizeof(int32_t));
    for (int t = 0; t < T; ++t)
        for (int j = 0; j < cnt[t]; ++j) count[ids[t * k + j]]++;
    group_start[0] = 0;
    for (int e = 0; e < E; ++e) group_start[e + 1] = group_start[e] + count[e];
    int nu = 0;
    for (int e = 0; e < E; ++e)
        if (count[e] > 0) uniq[nu++] = e;
    for (int e = 0; e < E; ++e) count[e] = 0;
    for (int i = 0; i < T * k; ++i) inv[i] = -1;
    for (int t = 0; t < T; ++t)
        for (int j = 0; j < cnt[t]; ++j) {
            int e = ids[t * k + j];
            int pos = group_start[e] + count[e]++;
            perm[pos] = t * k + j;
            inv[t * k + j] = pos;
        }
    free(count);
    return nu;
}

/* ---- whole layer ---------------------------------------------------------- */

static void expert_ffn(const uint8_t* blob, uint64_t gate_off, uint64_t up_off, uint64_t down_off,
                       int H, int I, int group, const float* x, float* y, float* g, float* u,
                       int threads) {
    /* decode.rs:333-336: gate, up, silu_mul, down */
    q4_gemv_mt(blob + gate_off, x, g, I, H, group, threads);
    q4_gemv_mt(blob + up_off, x, u, I, H, group, threads);
    lpo_silu_mul(g, u, g, I);
    q4_gemv_mt(blob + down_off, g, y, H, I, group, threads);
}

static int route(const lpo_layer* L, const float* logits, int32_t* ids, float* w) {
    if (L->gating == LPO_GATING_SIGMOID)
        return lpo_sigmoid_topk(logits, L->router_bias, L->experts, L->top_k, L->renorm,
                                L->routed_scaling, L->min_weight, ids, w);
    return lpo_top_k_softmax(logits, L->experts, L->top_k, L->renorm, ids, w);
}

int lpo_moe_layer(const lpo_layer* L, const float* x, float* h, int T,
                  const float* logits_in, float* logits_out, int32_t* ids_out,
                  float* w_out, int32_t* cnt_out, int wave, int threads) {
    const int H = L->hidden, I = L->inter, E = L->experts, k = L->top_k;
    int rc = 0;
    float* logits = (float*)malloc(sizeof(float) * (size_t)T * E);
    int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)T * k);
    float* w = (float*)malloc(sizeof(float) * (size_t)T * k);
    int32_t* cnt = (int32_t*)malloc(sizeof(int32_t) * (size_t)T);
    int maxi = I > L->shared_inter ? I : L->shared_inter;
    float* g = (float*)malloc(sizeof(float) * (size_t)maxi);
    float* u = (float*)malloc(sizeof(float) * (size_t)maxi);
    float* ys = (float*)malloc(sizeof(float) * (size_t)k * H);
    float* wsub = (float*)malloc(sizeof(float) * (size_t)k);
    uint8_t* in_wave = (uint8_t*)calloc((size_t)E, 1);
    uint8_t* used = (uint8_t*)calloc((size_t)E, 1);
    int32_t* uni = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);

    for (int t = 0; t < T; ++t) {
        float* lt = logits + (size_t)t * E;
        if (logits_in)
            memcpy(lt, logits_in + (size_t)t * E, sizeof(float) * (size_t)E);
        else
            lpo_router_logits(L->router_w, x + (size_t)t * H, lt, E, H);
        cnt[t] = route(L, lt, ids + (size_t)t * k, w + (size_t)t * k);
        for (int j = 0; j < cnt[t]; ++j) used[ids[t * k + j]] = 1;
    }
    /* decode.rs:483-485: sorted unique union */
    int nu = 0;
    for (int e = 0; e < E; ++e)
        if (used[e]) uni[nu++] = e;
    int ws = wave > 0 ? wave : (nu > 0 ? nu : 1);
    /* decode.rs:489-531: waves of the union; per token the picks inside the
     * wave in pick order, summed then added into h once per wave */
    for (int w0 = 0; w0 < nu && rc == 0; w0 += ws) {
        int w1 = w0 + ws < nu ? w0 + ws : nu;
        memset(in_wave, 0, (size_t)E);
        for (int i = w0; i < w1; ++i) in_wave[uni[i]] = 1;
        for (int t = 0; t < T && rc == 0; ++t) {
            int ns = 0;
            for (int j = 0; j < cnt[t]; ++j) {
                int e = ids[t * k + j];
                if (!in_wave[e]) continue;
                if (!L->blobs[e]) { rc = -1; break; }
                expert_ffn(L->blobs[e], L->gate_off, L->up_off, L->down_off, H, I, L->group,
                           x + (size_t)t * H, ys + (size_t)ns * H, g, u, threads);
                wsub[ns++] = w[t * k + j];
            }
            if (ns > 0 && rc == 0) lpo_moe_reduce(ys, wsub, h + (size_t)t * H, ns, H);
        }
    }
    /* kimi.rs:739-744, 779: the shared MLP, added unweighted after the routed part */
    if (rc == 0 && L->shared_blob) {
        for (int t = 0; t < T; ++t) {
            expert_ffn(L->shared_blob, L->sh_gate_off, L->sh_up_off, L->sh_down_off, H,
                       L->shared_inter, L->shared_group, x + (size_t)t * H, ys, g, u, threads);
            lpo_add(h + (size_t)t * H, ys, H);
        }
    }
    if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t)T * E);
    if (ids_out) memcpy(ids_out, ids, sizeof(int32_t) * (size_t)T * k);
    if (w_out) memcpy(w_out, w, sizeof(float) * (size_t)T * k);
    if (cnt_out) memcpy(cnt_out, cnt, sizeof(int32_t) * (size_t)T);
    free(logits); free(ids); free(w); free(cnt); free(g); free(u); free(ys); free(wsub);
    free(in_wave); free(used); free(uni);
    return rc;
}

/* ---- the rest of the decode step: CPU forms of the checks at
 * crates/llmpager-bench/src/kernels_bench.rs:60-256 (decode.cu semantics) ---- */

/* IEEE binary16, round to nearest even (what __float2half does in
 * kv_append_f16, decode.cu:242-261). */
uint16_t lpo_f32_to_f16_rne(float x) {
    uint32_t b = f2u(x);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    uint32_t a = b & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (a > 0x7F800000u ? 0x200u : 0u));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520: inf */
    if (a < 0x38800000u) {                                   /* below the f16 normal range */
        if (a < 0x33000000u) return sign;                    /* <= 2^-25: rounds to 0 */
        uint32_t e = a >> 23;
        uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126 - e; /* value = m * 2^(e-150); f16 subnormal unit = 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = a + 0xFFFu + ((a >> 13) & 1u);
    r -= 0x38000000u; /* rebias 127 -> 15 */
    return (uint16_t)(sign | (r >> 13));
}

/* kernels_bench.rs:64-101 (decode.cu:17-41): ms = sum(v*v)/n, inv =
 * 1/sqrt(ms + eps), y = x*inv*w, per row. */
void lpo_rmsnorm(const float* x, const float* w, float* y, int rows, int n, float eps) {
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * n;
        float ms = -0.0f;
        for (int i = 0; i < n; ++i) ms += xr[i] * xr[i];
        ms /= (float)n;
        const float inv = 1.0f / sqrtf(ms + eps);
        for (int i = 0; i < n; ++i) y[(size_t)r * n + i] = xr[i] * inv * w[i];
    }
}

/* kernels_bench.rs:104-113 (decode.cu:44-53) */
void lpo_scale_add(float* a, const float* b, float s, int n) {
    for (int i = 0; i < n; ++i) a[i] = a[i] + s * b[i];
}

/* kernels_bench.rs:116-135 (decode.cu:57-77, 242-261) */
void lpo_kv_append(const float* k, const float* v, void* kcache, void* vcache, int kv_heads, int head_dim,
                   int pos, int max_seq, int f16) {
    for (int h = 0; h < kv_heads; ++h)
        for (int d = 0; d < head_dim; ++d) {
            const size_t dst = ((size_t)h * max_seq + pos) * head_dim + d;
            const size_t src = (size_t)h * head_dim + d;
            if (f16) {
                ((uint16_t*)kcache)[dst] = lpo_f32_to_f16_rne(k[src]);
                ((uint16_t*)vcache)[dst] = lpo_f32_to_f16_rne(v[src]);
            } else {
                ((float*)kcache)[dst] = k[src];
                ((float*)vcache)[dst] = v[src];
            }
        }
}

/* kernels_bench.rs:171-192 (decode.cu:145-167, NeoX rotate-half): freq =
 * base^(-2i/hd), (s, c) = sin_cos(pos * freq). */
void lpo_rope(float* x, int heads, int head_dim, int pos, float base) {
    const int half = head_dim / 2;
    for (int h = 0; h < heads; ++h)
        for (int i = 0; i < half; ++i) {
            const float freq = powf(base, -2.0f * (float)i / (float)head_dim);
            const float ang = (float)pos * freq;
            const float s = sinf(ang), c = cosf(ang);
            float* p = x + (size_t)h * head_dim;
            const float x1 = p[i], x2 = p[i + half];
            p[i] = x1 * c - x2 * s;
            p[i + half] = x1 * s + x2 * c;
        }
}

static float cache_val(const void* c, size_t i, int f16) {
    return f16 ? lpo_f16_to_f32(((const uint16_t*)c)[i]) : ((const float*)c)[i];
}

/* One query against rows [0, seq) of a cache (row stride `stride`): scores
 * sum_d q[d]*k[d] (sequential) times scale; m = fold(f32::MIN, max); e =
 * exp(s - m); z = sum e; out[d] = sum_p e_p / z * v[p][d]
 * (kernels_bench.rs:205-220, 284-298). */
static void attend(const float* q, const void* k, const void* v, size_t kv_off, int stride, int dot_dim,
                   int out_dim, int seq, float scale, int f16, float* out, float* e) {
    float m = -3.40282347e+38f;
    for (int p = 0; p < seq; ++p) {
        float dot = -0.0f;
        for (int d = 0; d < dot_dim; ++d) dot += q[d] * cache_val(k, kv_off + (size_t)p * stride + d, f16);
        e[p] = dot * scale;
        m = e[p] > m ? e[p] : m;
    }
    float z = -0.0f;
    for (int p = 0; p < seq; ++p) {
        e[p] = expf(e[p] - m);
        z += e[p];
    }
    for (int d = 0; d < out_dim; ++d) {
        float acc = -0.0f;
        for (int p = 0; p < seq; ++p) acc += e[p] / z * cache_val(v, kv_off + (size_t)p * stride + d, f16);
        out[d] = acc;
    }
}

/* kernels_bench.rs:195-249 (decode.cu:172-325): GQA decode attention over
 * caches [kv_heads, max_seq, head_dim], f32 or IEEE half. */
void lpo_attn_decode(const float* q, const void* kcache, const void* vcache, float* out, int heads, int kv_heads,
                     int head_dim, int seq_len, int max_seq, float scale, int f16) {
    float* e = (float*)malloc(sizeof(float) * (size_t)(seq_len > 0 ? seq_len : 1));
    for (int h = 0; h < heads; ++h) {
        const int kv = h / (heads / kv_heads);
        attend(q + (size_t)h * head_dim, kcache, vcache, (size_t)kv * max_seq * head_dim, head_dim, head_dim,
               head_dim, seq_len, scale, f16, out + (size_t)h * head_dim, e);
    }
    free(e);
}

/* kernels_bench.rs:250-256 (decode.cu:328-339) */
void lpo_bf16_row(const uint16_t* table, int row, int n, float* out) {
    for (int i = 0; i < n; ++i) out[i] = lpo_bf16_to_f32(table[(size_t)row * n + i]);
}

/* ---- MLA: CPU forms of kernels_bench.rs:258-351 (mla.cu semantics) ---- */

/* kernels_bench.rs:258-282 (mla.cu:22-45) */
void lpo_mla_rope(float* x, int n_vecs, int stride, int offset, int half, int pos, const float* inv_freq,
                  float mscale) {
    for (int v = 0; v < n_vecs; ++v)
        for (int i = 0; i < half; ++i) {
            const float ang = (float)pos * inv_freq[i];
            const float s = sinf(ang) * mscale, c = cosf(ang) * mscale;
            float* p = x + (size_t)v * stride + offset + 2 * i;
            const float x1 = p[0], x2 = p[1];
            p[0] = x1 * c - x2 * s;
            p[1] = x1 * s + x2 * c;
        }
}

/* kernels_bench.rs:284-310 (mla.cu:51-111): MQA over one latent cache
 * [seq, qk_dim] (f32, or bf16 when cache_bf16), ctx [heads, c_dim].  Heads
 * in parallel over `threads`. */
void lpo_mla_attn_decode(const float* q, const void* cache, int cache_bf16, float* ctx, int heads, int qk_dim,
                         int c_dim, int seq_len, float scale, int threads) {
    if (cache_bf16) {
        /* widen once: the bf16 values are exact in f32 */
        float* wide = (float*)malloc(sizeof(float) * (size_t)seq_len * qk_dim);
        for (size_t i = 0; i < (size_t)seq_len * qk_dim; ++i) wide[i] = lpo_bf16_to_f32(((const uint16_t*)cache)[i]);
        lpo_mla_attn_decode(q, wide, 0, ctx, heads, qk_dim, c_dim, seq_len, scale, threads);
        free(wide);
        return;
    }
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int h = 0; h < heads; ++h) {
        float* e = (float*)malloc(sizeof(float) * (size_t)(seq_len > 0 ? seq_len : 1));
        attend(q + (size_t)h * qk_dim, cache, cache, 0, qk_dim, qk_dim, c_dim, seq_len, scale, 0,
               ctx + (size_t)h * c_dim, e);
        free(e);
    }
}

/* kernels_bench.rs:313-330 (mla.cu:120-148) */
void lpo_bf16_gemv_batch(const uint16_t* w, uint64_t w_stride, const float* x, int x_stride, float* y,
                         int y_stride, int rows, int cols, int batch) {
    for (int b = 0; b < batch; ++b)
        for (int r = 0; r < rows; ++r) {
            const uint16_t* wr = w + (size_t)b * w_stride + (size_t)r * cols;
            const float* xb = x + (size_t)b * x_stride;
            float acc = -0.0f;
            for (int c = 0; c < cols; ++c) acc += lpo_bf16_to_f32(wr[c]) * xb[c];
            y[(size_t)b * y_stride + r] = acc;
        }
}

/* kernels_bench.rs:332-344 (mla.cu:153-166) */
void lpo_strided_copy(const float* src, int src_stride, int src_off, float* dst, int dst_stride, int dst_off,
                      int n_vecs, int n) {
    for (int v = 0; v < n_vecs; ++v)
        for (int i = 0; i < n; ++i)
            dst[(size_t)v * dst_stride + dst_off + i] = src[(size_t)v * src_stride + src_off + i];
}
