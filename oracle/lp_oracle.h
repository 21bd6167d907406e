/*
 * lp_oracle.h -- CPU restatement of llmpager's MoE-layer hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or the timed CPU baseline), never as the thing measured or shipped.
 *
 * Every function restates the reference (glennswest/llmpager v0.21.0, Rust +
 * CUDA) and cites the file:line it follows, relative to the reference
 * checkout.  Arithmetic follows the reference's CPU forms: f32 throughout,
 * no fused multiply-add unless stated (the library is built with
 * -ffp-contract=off, matching rustc, which never contracts).
 */
#ifndef LP_ORACLE_H
#define LP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions ------------------------------------------------ */

/* f32 -> f16 bits exactly as crates/llmpager-core/src/quant.rs:151-171,
 * including its rounding quirk: the rounding carry is OR-ed (not added) into
 * the exponent, and ties round half-up. */
uint16_t lpo_f32_to_f16_ref(float x);
/* f16 bits -> f32, quant.rs:173-189 (exact). */
float lpo_f16_to_f32(uint16_t h);
float lpo_bf16_to_f32(uint16_t h);

/* libm expf: what Rust's f32::exp lowers to on the reference host (glibc). */
float lpo_expf(float x);
/* out[i] = expf(bits_to_float(first + i*stride)) for i < n: the checker for
 * exhaustive / strided sweeps over float bit patterns. */
void lpo_expf_sweep(uint32_t first, uint32_t stride, size_t n, float* out);

/* ---- q4 group-wise format (quant.rs) ----------------------------------- */

/* quant.rs:20-22 */
size_t lpo_q4_bytes(size_t rows, size_t cols, size_t group);
/* quant.rs:37-76.  Returns 0 on success, -1 on bad dimensions. */
int lpo_q4_quantize(const float* src, size_t rows, size_t cols, size_t group,
                    uint8_t* dst, size_t dst_len, float* max_err);
/* quant.rs:81-100 */
void lpo_q4_store_group(uint8_t* dst, size_t rows, size_t cols, size_t group,
                        size_t row, size_t g, float scale, const uint8_t* qs);
/* quant.rs:117-147.  Returns 0 on success, -1 on bad dimensions. */
int lpo_q4_dequantize(const uint8_t* buf, size_t buf_len, size_t rows,
                      size_t cols, size_t group, float* out);

/* ---- the hot-path kernels' CPU forms ------------------------------------ */

/* y = W x for one q4 region, in the reference's CPU checking form
 * (crates/llmpager-bench/src/gemv_bench.rs:30-41): dequantise each value to
 * f32 ((q-8)*scale, exact), multiply by x in f32, sum sequentially in f32. */
void lpo_q4_gemv(const uint8_t* region, const float* x, float* y, int rows,
                 int cols, int group);
/* Batched form with the semantics of q4g64_gemv_batch
 * (crates/llmpager-cuda/kernels/q4g64.cu:19-32): expert e reads
 * blobs[e] + region_off, x + e*x_stride, and writes y + e*rows. */
void lpo_q4_gemv_batch(const uint8_t* const* blobs, uint64_t region_off,
                       const float* x, int x_stride, float* y, int rows,
                       int cols, int group, int experts);
/* y = W x, W bf16 [rows, cols]; CPU form of kernels_bench.rs:136-149. */
void lpo_bf16_gemv(const uint16_t* w, const float* x, float* y, int rows,
                   int cols);
/* out = g/(1+exp(-g))*u; CPU form kernels_bench.rs:152-161 (decode.cu:117-128). */
void lpo_silu_mul(const float* gate, const float* up, float* out, int n);
/* out[i] += sum_e wts[e]*eouts[e*n+i]; q4g64.cu:84-99 (sum in pick order,
 * then one add). */
void lpo_moe_reduce(const float* eouts, const float* wts, float* out,
                    int experts, int n);
/* a += b; decode.cu:131-140 */
void lpo_add(float* a, const float* b, int n);

/* ---- routing ------------------------------------------------------------ */

/* top_k_softmax, crates/llmpager-run/src/decode.rs:734-749.  Writes
 * min(k, E) picks; returns the count. */
int lpo_top_k_softmax(const float* logits, int E, int k, int renorm,
                      int32_t* ids, float* w);
/* sigmoid_topk, crates/llmpager-run/src/kimi.rs:1155-1186.  Returns the
 * number of picks kept (<= k). */
int lpo_sigmoid_topk(const float* logits, const float* bias, int E, int k,
                     int renorm, float scaling, float min_weight,
                     int32_t* ids, float* w);

/* Router logits in the build's canonical reduction order (the order the
 * HIP router kernel uses, so the two agree bit for bit): 64 lanes; lane l
 * takes 8-column chunks l, l+64, l+128, ... and accumulates
 * acc = fmaf(w, x, acc) over them in column order; then six butterfly
 * stages acc += acc[l ^ off] for off = 32, 16, 8, 4, 2, 1.  Requires
 * H % 8 == 0.  The reference's own GPU order (decode.cu:80-114) differs and
 * is tolerance-checked (1e-4, kernels_bench.rs:148-149). */
void lpo_router_logits(const uint16_t* w, const float* x, float* logits,
                       int E, int H);

/* ---- dispatch ----------------------------------------------------------- */

/* Canonical token->expert dispatch over T tokens with cnt[t] picks each
 * (ids row-major [T, k]): the (t, j) pairs stably grouped by expert id
 * ascending, then t ascending.  Writes group_start[E+1] (exclusive scan of
 * the per-expert counts), perm[P] = t*k + j in that order, inv[t*k + j] =
 * position of the pair in perm (-1 for j >= cnt[t]), uniq[] = experts with
 * a nonzero count, ascending.  Returns the unique count.  The union of
 * decode.rs:483-485 is uniq; the per-token pick order of decode.rs:502-506
 * is recovered through inv. */
int lpo_moe_dispatch(const int32_t* ids, const int32_t* cnt, int T, int k,
                     int E, int32_t* perm, int32_t* group_start,
                     int32_t* inv, int32_t* uniq);

/* ---- whole MoE layer ---------------------------------------------------- */

enum { LPO_GATING_SOFTMAX = 0, LPO_GATING_SIGMOID = 1 };

typedef struct lpo_layer {
    int hidden, inter, experts, top_k, group;
    int gating;          /* LPO_GATING_* */
    int renorm;          /* norm_topk_prob */
    float routed_scaling;  /* sigmoid gating only (kimi.rs:1178-1180) */
    float min_weight;      /* sigmoid gating only (kimi.rs:1181-1183) */
    const uint16_t* router_w;      /* bf16 [E, H] */
    const float* router_bias;      /* [E] (sigmoid gating) */
    const uint8_t* const* blobs;   /* E expert blobs (host), NULL = absent */
    uint64_t gate_off, up_off, down_off;
    const uint8_t* shared_blob;    /* shared-expert blob or NULL */
    int shared_inter, shared_group;
    uint64_t sh_gate_off, sh_up_off, sh_down_off;
} lpo_layer;

/* One MoE layer over T tokens, restating decode.rs:303-337 (one token),
 * decode.rs:469-531 (multi-token union in waves of `wave` experts; 0 means
 * one wave) and kimi.rs:739-779 (shared expert added after the routed
 * part).  x is [T, H] (the post-norm activations), h is [T, H] and is
 * updated in place.  logits_in, if non-NULL, replaces the router GEMV
 * (the "given identical fp32 router logits" contract).  Optional outputs:
 * logits_out [T, E], ids_out/w_out [T, k], cnt_out [T].  Returns 0, or -1 if
 * a routed expert has no blob. */
int lpo_moe_layer(const lpo_layer* L, const float* x, float* h, int T,
                  const float* logits_in, float* logits_out,
                  int32_t* ids_out, float* w_out, int32_t* cnt_out, int wave,
                  int threads);

/* ---- the rest of the decode step (kernels_bench.rs:60-256; decode.cu) --- */

/* IEEE round-to-nearest-even f32 -> f16 bits (__float2half). */
uint16_t lpo_f32_to_f16_rne(float x);
void lpo_rmsnorm(const float* x, const float* w, float* y, int rows, int n, float eps);
void lpo_scale_add(float* a, const float* b, float s, int n);
void lpo_kv_append(const float* k, const float* v, void* kcache, void* vcache, int kv_heads, int head_dim,
                   int pos, int max_seq, int f16);
void lpo_rope(float* x, int heads, int head_dim, int pos, float base);
void lpo_attn_decode(const float* q, const void* kcache, const void* vcache, float* out, int heads, int kv_heads,
                     int head_dim, int seq_len, int max_seq, float scale, int f16);
void lpo_bf16_row(const uint16_t* table, int row, int n, float* out);

/* ---- MLA absorbed decode (kernels_bench.rs:258-351; mla.cu) -------------- */

void lpo_mla_rope(float* x, int n_vecs, int stride, int offset, int half, int pos, const float* inv_freq,
                  float mscale);
void lpo_mla_attn_decode(const float* q, const void* cache, int cache_bf16, float* ctx, int heads, int qk_dim,
                         int c_dim, int seq_len, float scale, int threads);
void lpo_bf16_gemv_batch(const uint16_t* w, uint64_t w_stride, const float* x, int x_stride, float* y,
                         int y_stride, int rows, int cols, int batch);
void lpo_strided_copy(const float* src, int src_stride, int src_off, float* dst, int dst_stride, int dst_off,
                      int n_vecs, int n);

#ifdef __cplusplus
}
#endif
#endif
