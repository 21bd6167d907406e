/*
 * llmpager_hip.h -- C ABI of the MI355X (gfx950) MoE-layer hot path.
 *
 * Drop-in boundary for glennswest/llmpager's `llmpager-cuda` crate: the
 * device runtime (`driver::Cuda`, crates/llmpager-cuda/src/driver.rs), the
 * hot-path kernel launchers (`kernels::Kernels`, src/kernels.rs) and the
 * expert-slot bookkeeping the pager runs on (`cache::ExpertCache`,
 * crates/llmpager-core/src/cache.rs; `pager::Pager`, src/pager.rs).  Paths in
 * the citations are relative to the reference checkout.
 *
 * Conventions (kept from the reference):
 *   - Device pointers are uint64_t (driver.rs:10 `CUdeviceptr = u64`).
 *   - Every call returns int: 0 on success, a negative LP_E_* code, or a
 *     positive hipError_t; lp_last_error() gives this thread's message
 *     (driver.rs:20-27 turns every failure into an error string).
 *   - The caller owns every buffer it passes; the library never frees them.
 *     The context owns only its code objects (decode.rs:756-780 ownership).
 *   - Launches are asynchronous on the caller's stream; nothing syncs unless
 *     its name says so (`*_sync`, lp_sync*).
 *   - A context may be used from several threads after each calls
 *     lp_bind_thread (driver.rs:125-129).
 */
#ifndef LLMPAGER_HIP_H
#define LLMPAGER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lp_ctx lp_ctx;
typedef void* lp_stream; /* hipStream_t; NULL is the null stream */
typedef void* lp_event;  /* hipEvent_t */

enum {
    LP_OK = 0,
    LP_E_INVALID = -1,     /* bad argument */
    LP_E_UNSUPPORTED = -2, /* shape or layout the kernels do not accept */
    LP_E_LOAD = -3,        /* code object missing or unloadable */
    LP_E_NOT_READY = -4,   /* (not returned by lp_event_done, which returns 0) */
    LP_E_DEVICE = -5       /* a kernel reported an error flag */
};

/* This thread's last error message ("" if none). */
const char* lp_last_error(void);
/* Library version string. */
const char* lp_version(void);

/* ---- device runtime: driver::Cuda (driver.rs:29-304) --------------------- */

/* Cuda::init (driver.rs:66-112) + Kernels::load (kernels.rs:44-68): make
 * `device` current and load the gfx950 code objects from `hsaco_dir` with
 * hipModuleLoad (NULL: the directory the library was loaded from). */
int lp_init(int device, const char* hsaco_dir, lp_ctx** out);
/* Unload the code objects.  Never frees caller buffers. */
void lp_destroy(lp_ctx* ctx);
/* driver.rs:125-129: make the context's device current on this thread. */
int lp_bind_thread(lp_ctx* ctx);
/* driver.rs:117-123 */
int lp_mem_info(lp_ctx* ctx, uint64_t* free_bytes, uint64_t* total_bytes);
/* driver.rs:131-141 */
int lp_alloc_device(lp_ctx* ctx, size_t bytes, uint64_t* out);
int lp_free_device(lp_ctx* ctx, uint64_t ptr);
/* driver.rs:143-151 (page-locked host memory, hipHostMalloc) */
int lp_alloc_pinned(lp_ctx* ctx, size_t bytes, void** out);
int lp_free_pinned(lp_ctx* ctx, void* p);
/* driver.rs:153-163, 201-204 */
int lp_stream_create(lp_ctx* ctx, lp_stream* out);
int lp_stream_destroy(lp_ctx* ctx, lp_stream s);
int lp_event_create(lp_ctx* ctx, lp_event* out);
int lp_event_destroy(lp_ctx* ctx, lp_event e);
/* driver.rs:165-188: asynchronous copies on `s` */
int lp_htod_async(lp_ctx* ctx, uint64_t dst, const void* src, size_t bytes, lp_stream s);
int lp_dtoh_async(lp_ctx* ctx, void* dst, uint64_t src, size_t bytes, lp_stream s);
int lp_dtod_async(lp_ctx* ctx, uint64_t dst, uint64_t src, size_t bytes, lp_stream s);
int lp_memset_async(lp_ctx* ctx, uint64_t dst, int value, size_t bytes, lp_stream s);
/* driver.rs:190-199 */
int lp_record_event(lp_ctx* ctx, lp_event e, lp_stream s);
int lp_sync_event(lp_ctx* ctx, lp_event e);
/* event_done (driver.rs:206-213): 1 complete, 0 pending, <0 error. */
int lp_event_done(lp_ctx* ctx, lp_event e);
int lp_event_elapsed_ms(lp_ctx* ctx, lp_event start, lp_event end, float* ms);
/* driver.rs:216-219 */
int lp_stream_wait_event(lp_ctx* ctx, lp_stream s, lp_event e);
/* driver.rs:221-230 */
int lp_sync_stream(lp_ctx* ctx, lp_stream s);
int lp_sync(lp_ctx* ctx);

/* ---- hot-path launchers: kernels::Kernels (kernels.rs) ------------------- */

/* q4g64_gemv_batch (kernels.rs:102-127; q4g64.cu:19-81): for e < experts,
 * y[e*rows + r] = sum_g s[r,g] * sum_{c in g} (q[r,c] - 8) * x[e*x_stride + c],
 * reading the q4 region at ((u64*)blobs)[e] + region_off.  fp32 accumulation.
 * group must divide cols and be a multiple of 8. */
int lp_q4_gemv_batch(lp_ctx* ctx, uint64_t blobs, uint64_t region_off, uint64_t x, int x_stride,
                     uint64_t y, int rows, int cols, int group, int experts, lp_stream s);
/* q4g64_gemv (kernels.rs:73-95; q4g64.cu:101-161): one q4 region at `blob`. */
int lp_q4_gemv(lp_ctx* ctx, uint64_t blob, uint64_t x, uint64_t y, int rows, int cols, int group,
               lp_stream s);
/* moe_reduce (kernels.rs:131-144; q4g64.cu:84-99):
 * out[i] += sum_{e<experts} wts[e] * eouts[e*n + i], summed in order. */
int lp_moe_reduce(lp_ctx* ctx, uint64_t eouts, uint64_t wts, uint64_t out, int experts, int n,
                  lp_stream s);
/* silu_mul (kernels.rs:224-236; decode.cu:117-128): out = g/(1+exp(-g))*u. */
int lp_silu_mul(lp_ctx* ctx, uint64_t gate, uint64_t up, uint64_t out, int n, lp_stream s);
/* bf16_gemv (kernels.rs:202-222; decode.cu:80-114): y = W x, W bf16 [rows, cols]. */
int lp_bf16_gemv(lp_ctx* ctx, uint64_t w, uint64_t x, uint64_t y, int rows, int cols,
                 lp_stream s);
/* add (kernels.rs:239-250; decode.cu:131-140): a += b. */
int lp_add(lp_ctx* ctx, uint64_t a, uint64_t b, int n, lp_stream s);

/* ---- the rest of the decode step: kernels::Kernels (kernels.rs; decode.cu) -- */

/* rmsnorm (kernels.rs:145-158; decode.cu:17-41): per row r < rows,
 * y[r] = x[r] / sqrt(mean(x[r]^2) + eps) * w; y may be x. */
int lp_rmsnorm(lp_ctx* ctx, uint64_t x, uint64_t w, uint64_t y, int rows, int n, float eps, lp_stream s);
/* scale_add (kernels.rs:161-173; decode.cu:44-53): a += s * b. */
int lp_scale_add(lp_ctx* ctx, uint64_t a, uint64_t b, float s_, int n, lp_stream s);
/* kv_append (kernels.rs:176-196; decode.cu:57-77, 242-261): k, v
 * [kv_heads, head_dim] into caches [kv_heads, max_seq, head_dim] at pos;
 * f16 != 0: IEEE half caches (round to nearest even). */
int lp_kv_append(lp_ctx* ctx, uint64_t k, uint64_t v, uint64_t kcache, uint64_t vcache, int kv_heads,
                 int head_dim, int pos, int max_seq, int f16, lp_stream s);
/* rope (kernels.rs:252-266; decode.cu:145-167): NeoX rotate-half RoPE in
 * place over [heads, head_dim], theta_i = pos * base^(-2i/head_dim). */
int lp_rope(lp_ctx* ctx, uint64_t x, int heads, int head_dim, int pos, float base, lp_stream s);
/* attn_decode (kernels.rs:269-292; decode.cu:172-325): one query per head
 * [heads, head_dim] against caches [kv_heads, max_seq, head_dim] (f32, or
 * half when f16 != 0), GQA head -> kv head h / (heads / kv_heads),
 * positions < seq_len; scratch [heads, max_seq] f32 (split records). */
int lp_attn_decode(lp_ctx* ctx, uint64_t q, uint64_t kcache, uint64_t vcache, uint64_t out, uint64_t scratch,
                   int heads, int kv_heads, int head_dim, int seq_len, int max_seq, float scale, int f16,
                   lp_stream s);
/* bf16_row (kernels.rs:294-306; decode.cu:328-339): out[:n] = f32(table[row, :n]). */
int lp_bf16_row(lp_ctx* ctx, uint64_t table, int row, int n, uint64_t out, lp_stream s);

/* ---- the fused decode step ------------------------------------------------
 * No reference counterparts: each entry point does the arithmetic of launches
 * that Decoder::step (decode.rs:275-301) issues one by one, in one launch. */

/* rmsnorm + bf16_gemv (decode.rs:282-285, 359-360): y_i = W_i . rmsnorm(x, ln)
 * for up to three bf16 [rows_i, cols] matrices sharing x [cols] (rows1 = 0
 * and rows2 = 0 leave them out; ln = 0 skips the norm: y_i = W_i . x).
 * cols a multiple of 8, at most 4096; x and the matrices 16-byte aligned. */
int lp_rmsnorm_gemv(lp_ctx* ctx, uint64_t x, uint64_t ln, float eps, int cols, uint64_t w0, int rows0,
                    uint64_t y0, uint64_t w1, int rows1, uint64_t y1, uint64_t w2, int rows2, uint64_t y2,
                    lp_stream s);
/* bf16_gemv + add + rmsnorm (decode.rs:296-301): h[rows] += W . x (W bf16
 * [rows, cols]), then hn = rmsnorm(h, ln).  Same limits on cols as above.
 * Uses the stream's arrival counters (launches that overlap on one stream's
 * slot are not allowed; launches on one stream run in order). */
int lp_gemv_add_rmsnorm(lp_ctx* ctx, uint64_t w, uint64_t x, int rows, int cols, uint64_t h, uint64_t ln,
                        float eps, uint64_t hn, lp_stream s);
/* Per-head rmsnorm of q [heads, 128] with q_norm and of k [kv_heads, 128]
 * with k_norm (0: none), NeoX rope of both at pos, kv_append of k and v into
 * fp16 caches [kv_heads, max_seq, 128] at pos, and attn_decode over
 * positions 0..pos into out [heads, 128] (decode.rs:283-294).  q, k and v
 * are read only; scratch [heads, max_seq] f32.  heads / kv_heads in
 * {1, 2, 4, 8, 16}, kv_heads <= 16. */
int lp_attn_fused(lp_ctx* ctx, uint64_t q, uint64_t k, uint64_t v, uint64_t q_norm, uint64_t k_norm, float eps,
                  float rope_base, uint64_t kcache, uint64_t vcache, uint64_t out, uint64_t scratch, int heads,
                  int kv_heads, int head_dim, int pos, int max_seq, float scale, lp_stream s);
/* lp_attn_fused into att, then h[hidden] += W_o . att (W_o bf16 [hidden,
 * heads * 128]) and hn = rmsnorm(h, post_ln), in one launch (decode.rs:
 * 283-301): the o projection's workgroups load W_o while the attention
 * runs.  hidden and heads * 128 at most 4096.  Uses the stream's arrival
 * counters, like lp_gemv_add_rmsnorm. */
int lp_attn_block(lp_ctx* ctx, uint64_t q, uint64_t k, uint64_t v, uint64_t q_norm, uint64_t k_norm, float eps,
                  float rope_base, uint64_t kcache, uint64_t vcache, uint64_t att, uint64_t scratch, int heads,
                  int kv_heads, int head_dim, int pos, int max_seq, float scale, uint64_t wo, uint64_t h,
                  uint64_t post_ln, uint64_t hn, int hidden, lp_stream s);
/* The o projection's wait in lp_attn_block is bounded (about 30 ms): one
 * that gives up counts itself and lets the launch end with a wrong result
 * instead of hanging.  This waits for the device, returns the count since the
 * last call in *timeouts (0 normally) and clears it, with the fused step's
 * counters of each stream that had one. */
int lp_step_errors_sync(lp_ctx* ctx, int32_t* timeouts);

/* ---- MLA absorbed decode: kernels::Kernels (kernels.rs; mla.cu) ----------- */

/* mla_rope (kernels.rs:311-330; mla.cu:22-45): pairs (2i, 2i+1) of the
 * slice at `offset` of n_vecs vectors (stride apart) rotate by
 * pos * inv_freq[i] (device f32 [half]), both factors times mscale. */
int lp_mla_rope(lp_ctx* ctx, uint64_t x, int n_vecs, int stride, int offset, int half, int pos,
                uint64_t inv_freq, float mscale, lp_stream s);
/* mla_attn_decode (kernels.rs:333-354; mla.cu:51-111): MQA decode over one
 * f32 latent cache [max_seq, qk_dim] shared by all heads; scores use all
 * qk_dim of q [heads, qk_dim], ctx [heads, c_dim] the first c_dim columns;
 * scratch [heads, max_seq] f32. */
int lp_mla_attn_decode(lp_ctx* ctx, uint64_t q, uint64_t cache, uint64_t ctx_out, uint64_t scratch, int heads,
                       int qk_dim, int c_dim, int seq_len, int max_seq, float scale, lp_stream s);
/* bf16_gemv_batch (kernels.rs:357-381; mla.cu:120-148): y_b = W_b x_b with
 * W_b = w + b*w_stride bf16 [rows, cols], x_b = x + b*x_stride,
 * y_b = y + b*y_stride (strides in elements). */
int lp_bf16_gemv_batch(lp_ctx* ctx, uint64_t w, uint64_t w_stride, uint64_t x, int x_stride, uint64_t y,
                       int y_stride, int rows, int cols, int batch, lp_stream s);
/* strided_copy (kernels.rs:386-404; mla.cu:153-166). */
int lp_strided_copy(lp_ctx* ctx, uint64_t src, int src_stride, int src_off, uint64_t dst, int dst_stride,
                    int dst_off, int n_vecs, int n, lp_stream s);
/* Batched MLA decode over bf16 latent caches (no reference counterpart: the
 * reference calls mla_attn_decode once per sequence, kimi.rs:892-939):
 * q f32 [batch][heads][qk_dim]; sequence b's cache rows (bf16 [seq, qk_dim])
 * at cache + b * cache_stride bytes; seq_lens device i32 [batch], each in
 * 1..max_seq (a larger value is taken as max_seq: no row past a sequence's
 * max_seq rows is read); ctx_out f32 [batch][heads][c_dim].  heads <= 16, qk_dim =
 * 32 x {3,4,6,8,12,16,18,20}, c_dim a multiple of 64 up to 512.  The
 * workspace holds lp_mla_batch_ws_bytes(ctx, batch, c_dim, max_seq) bytes. */
uint64_t lp_mla_batch_ws_bytes(lp_ctx* ctx, int batch, int c_dim, int max_seq);
int lp_mla_attn_decode_batch(lp_ctx* ctx, uint64_t q, uint64_t cache, uint64_t cache_stride, uint64_t seq_lens,
                             uint64_t ctx_out, uint64_t workspace, int batch, int heads, int qk_dim, int c_dim,
                             int max_seq, float scale, lp_stream s);

/* ---- fused MoE layer ------------------------------------------------------ */

enum { LP_GATING_SOFTMAX = 0, LP_GATING_SIGMOID = 1 };

/* One MoE layer as the device sees it.  Blob layout per expert
 * (crates/llmpager-convert/src/lib.rs:245-286): a 32-byte header, then the
 * gate [inter, hidden], up [inter, hidden] and down [hidden, inter] q4
 * regions (quant.rs:1-22: f16 scales [rows, cols/group], then nibbles
 * [rows, cols/2], value q stored as q + 8).  Expert e lives at
 * arena_base + slot_table[e] * slot_span (pager.rs:310-318); slot -1 means
 * not resident. */
typedef struct lp_moe_layer_desc {
    int32_t hidden;         /* H (model.rs:34 hidden_size) */
    int32_t inter;          /* I (moe_intermediate_size) */
    int32_t experts;        /* E routed experts (<= 1024) */
    int32_t top_k;          /* k (<= 16) */
    int32_t group;          /* q4 group (32 or 64, any multiple of 32) */
    int32_t gating;         /* LP_GATING_SOFTMAX (decode.rs:734-749) or
                               LP_GATING_SIGMOID (kimi.rs:1155-1186) */
    int32_t renorm;         /* norm_topk_prob (model.rs:46; kimi.rs:123) */
    float routed_scaling;   /* sigmoid gating only (kimi.rs:122) */
    float min_weight;       /* sigmoid gating only (kimi.rs:1181-1183) */
    int32_t reserved0;
    uint64_t router_w;      /* device bf16 [E, H] (model.rs:80, 183) */
    uint64_t router_bias;   /* device f32 [E] (sigmoid gating) or 0 */
    uint64_t slot_table;    /* device int32 [E] */
    uint64_t arena_base;    /* device address of slot 0 */
    uint64_t slot_span;     /* bytes per slot (pager.rs:263) */
    uint64_t gate_off, up_off, down_off; /* region offsets in a blob (decode.rs:183-185) */
    /* The always-on shared MLP (kimi.rs:739-744, added unweighted after the
     * routed part at kimi.rs:779; one MLP whose width is the shared experts'
     * combined intermediate size, kimi.rs:274-291).  shared_blob = 0: none. */
    uint64_t shared_blob;   /* device address of the shared MLP's blob */
    int32_t shared_inter;   /* its intermediate size */
    int32_t shared_group;   /* its q4 group */
    uint64_t sh_gate_off, sh_up_off, sh_down_off; /* region offsets in that blob */
} lp_moe_layer_desc;

/* Byte offsets of the workspace parts for T tokens (all 256-byte aligned). */
typedef struct lp_moe_ws_layout {
    uint64_t logits;  /* f32 [T, E] router logits */
    uint64_t ids;     /* i32 [T, k] picked expert ids in pick order, -1 past cnt */
    uint64_t wts;     /* f32 [T, k] routing weights in pick order */
    uint64_t cnt;     /* i32 [T] picks per token */
    uint64_t gs;      /* i32 [E+1] dispatch group starts */
    uint64_t perm;    /* i32 [T*k] pick index t*k+j per dispatch position */
    uint64_t inv;     /* i32 [T*k] dispatch position per pick, -1 if unused */
    uint64_t uniq;    /* i32 [E] experts with picks, ascending */
    uint64_t meta;    /* i32 [16]: [0] unique count, [1] error flags */
    uint64_t et;      /* 32-byte expert entries [E] for the grouped kernels */
    uint64_t act;     /* f32 [T*k, I]; on the prefill GEMM path i32 [T*k][ceil(I/128)], the
                         exponent of each 128-column chunk of the act images in actimg */
    uint64_t y;       /* f32 [T*k, H] */
    uint64_t xf;      /* [T] fp16 images of x for the prefill GEMM, each row scaled by 2^-xexp[t]
                         (size 0 without it) */
    uint64_t xd;      /* [T] digit images of x for the grouped kernels (per 32 columns 16-bit
                         fixed point as two int8 digits, a seed and a scale) */
    uint64_t sh_et;   /* shared MLP: its expert entry (size 0 without one) */
    uint64_t sh_perm; /* shared MLP: i32 [T] identity token list */
    uint64_t sh_act;  /* shared MLP: f32 [T, shared_inter] */
    uint64_t sh_y;    /* shared MLP: f32 [T, H] */
    uint64_t tiles;   /* prefill GEMM tile list (size 0 on the decode path) */
    uint64_t actimg;  /* prefill GEMM: fp16 images of the act rows (size 0 on the decode path) */
    uint64_t xexp;    /* i32 [T]: prefill GEMM: the power-of-two exponent of each token's image in xf */
    uint64_t disp;    /* dispatch scratch of batches above 64 tokens */
    uint64_t total;   /* bytes */
} lp_moe_ws_layout;

int lp_moe_ws_layout_get(const lp_moe_layer_desc* d, int T, lp_moe_ws_layout* out);

/* Every entry point below that takes a workspace also takes its size in
 * bytes (ws_bytes) and refuses, before any launch, a workspace that is null,
 * not 256-byte aligned or smaller than lp_moe_ws_layout_get(d, T).total (for
 * a stack: than the largest layer's).  This is that check on its own, with no
 * context and no device: LP_OK, or the error the entry points would give.
 * (No counterpart in the reference, whose engine sizes its buffers itself,
 * decode.rs:165-199.) */
int lp_moe_workspace_check(const lp_moe_layer_desc* layers, int n_layers, int T, uint64_t workspace,
                           uint64_t ws_bytes);

/* Routing for T tokens without the host round trip of decode.rs:305-331:
 * router logits (T <= 64: GEMV in the canonical fp32 FMA order; larger T: an
 * MFMA GEMM over exact products, equal to fp32 rounding), softmax or sigmoid
 * top-k with glibc-exact expf (bit-exact with the reference's host routing
 * given the same logits), and the stable token->expert dispatch.
 * x: f32 [T, H], 16-byte aligned. */
int lp_moe_route(lp_ctx* ctx, const lp_moe_layer_desc* d, uint64_t x, int T, uint64_t workspace,
                 uint64_t ws_bytes, lp_stream s);
/* Routing from caller-supplied logits (f32 [T, E], copied into the
 * workspace): the "given identical fp32 router logits" contract. */
int lp_moe_route_logits(lp_ctx* ctx, const lp_moe_layer_desc* d, uint64_t logits, int T,
                        uint64_t workspace, uint64_t ws_bytes, lp_stream s);
/* Expert half of the layer after lp_moe_route*: fragment images of x,
 * grouped gate/up + SiLU, grouped down, and h[t] += sum_j w[t][j] * y[t][j]
 * in pick order.  x and h 16-byte aligned. */
int lp_moe_experts(lp_ctx* ctx, const lp_moe_layer_desc* d, uint64_t x, uint64_t h, int T,
                   uint64_t workspace, uint64_t ws_bytes, lp_stream s);
/* One wave of a paged multi-token step (decode.rs:483-531; Kimi
 * kimi.rs:965-1021): when a layer's union of picked experts exceeds its slots,
 * the reference fetches it in waves (`union.chunks(wave)`, the union sorted by
 * expert id) and, per wave, adds each token's picks inside the wave, summed in
 * pick order, into h once.  After lp_moe_route* (and, per wave, the pager's
 * requests for the wave's experts and lp_moe_resolve): the routed experts
 * uniq[u_first, u_first + u_count) of the dispatch's unique list (the `uniq`
 * part of the workspace, ascending ids; its length is meta[0]) are computed
 * and h[t] += sum over token t's picks among them; tokens with none are left
 * as they are.  with_shared != 0 also adds the shared MLP's output after the
 * routed sum (pass it with the last wave, as the reference adds the shared
 * MLP after the routed part, kimi.rs:779).  x must not be h (every wave reads
 * the same input); decode batches only (T <= 64). */
int lp_moe_experts_wave(lp_ctx* ctx, const lp_moe_layer_desc* d, uint64_t x, uint64_t h, int T, uint64_t workspace,
                        uint64_t ws_bytes, int u_first, int u_count, int with_shared, lp_stream s);
/* Paged flow (decode.rs:305-331 order: route, then request the picks, then
 * compute): after lp_moe_route* and the pager's requests for the picked
 * experts, re-resolve the expert table's blob addresses through the layer's
 * now-current slot table, before lp_moe_experts. */
int lp_moe_resolve(lp_ctx* ctx, const lp_moe_layer_desc* d, int T, uint64_t workspace, uint64_t ws_bytes,
                   lp_stream s);
/* The whole layer (decode.rs:303-337 for one token, 469-531 for many):
 * lp_moe_route followed by lp_moe_experts, with the fragment images of x
 * written by the router kernel.  h: f32 [T, H], updated in place. */
int lp_moe_forward(lp_ctx* ctx, const lp_moe_layer_desc* d, uint64_t x, uint64_t h, int T,
                   uint64_t workspace, uint64_t ws_bytes, lp_stream s);
/* The layer-stack driver (decode.rs:277-343 restricted to the MoE block;
 * the batched layer loop decode.rs:431-532): lp_moe_forward over
 * layers[0 .. n_layers), in order, the layer input being the residual itself
 * (x = h; the router and expert GEMVs read h, the combine updates it in
 * place).  One workspace serves every layer: size it for the largest
 * lp_moe_ws_layout of the stack.  Every descriptor is checked before the
 * first launch.  No host synchronisation between layers (the reference reads
 * the router logits back and syncs once per layer, decode.rs:306-307). */
int lp_moe_stack_forward(lp_ctx* ctx, const lp_moe_layer_desc* layers, int n_layers, uint64_t h, int T,
                         uint64_t workspace, uint64_t ws_bytes, lp_stream s);
/* The same stack captured once into a HIP graph (no counterpart in the
 * reference, whose launches are issued one by one from the host): every
 * kernel node keeps the arguments given here (h, T, workspace, the
 * descriptors' tables), so a replay reruns exactly this stack.  s must be a
 * created stream (the null stream cannot be captured).  The graph holds a
 * set of the routing kernels' arrival counters of its own until
 * lp_graph_destroy (so s may be destroyed, and other streams may route, while
 * it lives): replays of one graph must not overlap one another.  Destroy
 * graphs before their context; lp_graph_destroy waits for the device first.
 * The graph holds no memset nodes. */
typedef struct lp_graph lp_graph;
int lp_moe_stack_capture(lp_ctx* ctx, const lp_moe_layer_desc* layers, int n_layers, uint64_t h, int T,
                         uint64_t workspace, uint64_t ws_bytes, lp_stream s, lp_graph** out);
/* The general form (no counterpart in the reference, whose decode step,
 * decode.rs:263-363, issues each launch from the host every step): every
 * launch this library makes on s between lp_graph_capture_begin and
 * lp_graph_capture_end (the 1:1 kernels of the attention block, fused MoE
 * layers, stacks through lp_moe_stack_forward) becomes one graph, with the
 * arguments given then (a decode step at one position replays at that
 * position).  The graph owns a set of routing arrival counters as
 * lp_moe_stack_capture's does.  One capture per context at a time; s must be
 * a created stream; copies, memsets and synchronisation are not allowed in
 * between, and lp_moe_stack_capture is refused. */
int lp_graph_capture_begin(lp_ctx* ctx, lp_stream s);
int lp_graph_capture_end(lp_ctx* ctx, lp_stream s, lp_graph** out);
int lp_graph_launch(lp_ctx* ctx, lp_graph* g, lp_stream s);
void lp_graph_destroy(lp_graph* g);
/* lp_moe_forward without a workspace argument and without any allocation:
 * no counterpart in the reference.  For callers that cannot call hipMalloc
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).  The workspace is a file-scope device array of
 * LP_NOALLOC_SCRATCH_BYTES per device, held until the process ends; a layer
 * whose lp_moe_ws_layout total exceeds it gets LP_E_UNSUPPORTED.  Every call
 * on a device shares that device's array: calls that overlap on one device
 * (different streams or unordered threads) race, so callers serialise them.
 * The routing tables a call leaves in the array are those of the last call. */
#define LP_NOALLOC_SCRATCH_BYTES (16ull << 20)
int lp_moe_forward_noalloc(lp_ctx* ctx, const lp_moe_layer_desc* d, uint64_t x, uint64_t h, int T,
                           lp_stream s);
/* LP_NOALLOC_SCRATCH_BYTES, as built into the library. */
uint64_t lp_noalloc_scratch_bytes(void);
/* Synchronising readback of meta[0..1] (unique count, error flags). */
int lp_moe_status_sync(lp_ctx* ctx, uint64_t workspace, uint64_t ws_bytes, const lp_moe_layer_desc* d, int T,
                       lp_stream s, int32_t* unique_count, int32_t* error_flags);

/* ---- expert-slot bookkeeping: cache::ExpertCache (cache.rs:58-241) -------- */

typedef struct lp_cache lp_cache;
enum { LP_LOOKUP_HIT = 0, LP_LOOKUP_MISS = 1, LP_LOOKUP_STALLED = 2 };

/* cache.rs:71-73 (ExpertCache::new) and :78-102 (partitioned).  NULL on a
 * zero argument (the reference asserts). */
lp_cache* lp_cache_new(uint16_t num_layers, uint32_t slots_per_layer, uint32_t decay_interval);
lp_cache* lp_cache_partitioned(uint32_t partitions, uint32_t ids_per_partition,
                               uint32_t slots_per_partition, uint32_t decay_interval);
void lp_cache_free(lp_cache* c);
/* cache.rs:106-108 */
uint32_t lp_cache_fold(uint16_t layer, uint16_t expert, uint32_t experts_per_layer);
/* cache.rs:112-118 */
uint32_t lp_cache_slots_per_partition(const lp_cache* c);
uint32_t lp_cache_total_slots(const lp_cache* c);
/* cache.rs:132-179: returns LP_LOOKUP_HIT / MISS / STALLED; the slot is
 * pinned on HIT and MISS; *evicted is the displaced id or -1. */
int lp_cache_acquire(lp_cache* c, uint32_t id, uint32_t* slot, int64_t* evicted);
/* cache.rs:184-195: 1 (pinned hit on a published slot) or 0. */
int lp_cache_lookup_ready(lp_cache* c, uint32_t id, uint32_t* slot);
/* cache.rs:198-204 */
int lp_cache_publish(lp_cache* c, uint32_t slot);
int lp_cache_is_ready(const lp_cache* c, uint32_t slot);
/* cache.rs:207-211: LP_E_INVALID for a release without a matching acquire. */
int lp_cache_release(lp_cache* c, uint32_t slot);
/* cache.rs:218-225 */
int lp_cache_decay_all(lp_cache* c);
/* cache.rs:229-236: 1 when every slot the id could use is pinned and ready. */
int lp_cache_is_wedged(const lp_cache* c, uint32_t id);
/* cache.rs:238-240 */
int lp_cache_stats(const lp_cache* c, uint64_t* hits, uint64_t* misses);
/* The id a slot holds, or -1 (no counterpart in the reference: lets a caller
 * rebuild a layer's device slot table from the cache). */
int64_t lp_cache_slot_id(const lp_cache* c, uint32_t slot);

/* ---- expert pager: pager::Pager (crates/llmpager-cuda/src/pager.rs) ------ */

typedef struct lp_pager lp_pager;

/* Where missed experts are copied from (pager.rs:650-718 reads a pack into a
 * pinned staging buffer on I/O worker threads, then copies it to the slot). */
enum {
    LP_PAGER_SRC_PINNED = 0, /* host_blobs is pinned: copies go straight from it */
    LP_PAGER_SRC_HOST = 1,   /* host_blobs is pageable (a RAM tier, a mapped file): workers stage
                                each blob through a pinned ring, then copy it */
    LP_PAGER_SRC_PACK = 2    /* a .llmpk pack (lp_pager_open): workers pread into the ring */
};

typedef struct lp_pager_config {
    uint32_t layers;            /* pack layers (pager.rs:263-264) */
    uint32_t experts_per_layer; /* ids fold (layer, expert) on this (pager.rs:224-226) */
    uint32_t slots_per_layer;   /* PagerConfig::slots_per_layer (pager.rs:34) */
    uint32_t decay_interval;    /* per-layer pools: halve counters every this many inserts (:37) */
    uint64_t blob_bytes;        /* bytes copied per miss */
    uint64_t span;              /* VRAM bytes per slot; 0 = blob_bytes rounded up to 4096 (:263) */
    const void* host_blobs;     /* PINNED / HOST sources: blob (l, e) at host_blobs + (l*E + e)*host_stride */
    uint64_t host_stride;
    int32_t copy_streams;       /* PINNED source: 1..8 copy streams */
    int32_t global_pool;        /* one pool for every layer (LLMPAGER_GLOBAL_POOL, :296-318) */
    uint32_t pool_decay_tokens; /* global pool: decay every this many ticks; 0 = 4 (:361-365) */
    int32_t source;             /* LP_PAGER_SRC_* */
    int32_t direct;             /* pack reads with O_DIRECT (PagerConfig::direct, :38-41) */
    uint32_t io_threads;        /* HOST / PACK: I/O workers, each with its own copy stream
                                   (PagerConfig::io_threads, :35); 0 = 4 */
    uint32_t ring_slots;        /* pinned staging buffers of one span per worker; 0 = 2 */
    uint32_t stage_threads;     /* threads sharing one blob's staging copy or read; 0 = 4 */
    uint64_t ram_bytes;         /* PACK: host-RAM expert tier in bytes, 0 = none (PagerConfig::ram_bytes, :42-45) */
    uint64_t reserve_bytes;     /* device memory to leave free, 0 = none (PagerConfig::reserve_bytes, :46-50):
                                   slots_per_layer is lowered until the arena and slot tables leave this much
                                   free (lp_pager_slots_per_layer gives the result); refused if not even one
                                   slot per layer fits */
} lp_pager_config;

typedef struct lp_pager_metrics {
    uint64_t hits, misses, bytes_fetched, fetches, stalls; /* pager.rs:568-589 (Metrics) */
    uint64_t ram_hits;                                     /* fills served by the RAM tier */
    uint64_t latency_ms_buckets[7]; /* worker fetches' read-and-enqueue time: <1, <2, <5, <10, <20, <50,
                                       >=50 ms (pager.rs:677-686; zero for the pinned source) */
} lp_pager_metrics;

/* ExpertHandle (pager.rs:169-178): a pinned, resident or in-flight expert. */
typedef struct lp_expert_handle {
    uint16_t layer, expert;
    uint32_t slot;
    uint64_t dev;  /* device address of the expert's blob */
    uint64_t len;  /* valid bytes */
} lp_expert_handle;

/* Pager::new (pager.rs:260-388) over host memory (PINNED or HOST source): one
 * arena of layers x slots_per_layer slots, per-layer device slot tables
 * (expert -> global slot, -1 absent), copy streams or I/O workers. */
int lp_pager_new(lp_ctx* ctx, const lp_pager_config* cfg, lp_pager** out);
/* Pager::new(cuda, &Path, cfg) (pager.rs:260-388) over a .llmpk pack: layers,
 * experts and the span come from the pack (cfg's must be 0 or equal); reads
 * by cfg->io_threads workers into pinned staging rings, O_DIRECT when
 * cfg->direct, through a RAM tier of cfg->ram_bytes. */
int lp_pager_open(lp_ctx* ctx, const char* pack_path, const lp_pager_config* cfg, lp_pager** out);
/* Drop (pager.rs:606-620): waits for copies in flight, frees the arena. */
void lp_pager_free(lp_pager* p);
/* The arena base (the layer desc's arena_base), the slot span (its
 * slot_span) and layer l's device slot table (its slot_table). */
uint64_t lp_pager_arena(const lp_pager* p);
uint64_t lp_pager_span(const lp_pager* p);
uint64_t lp_pager_slot_table(const lp_pager* p, uint32_t layer);
uint32_t lp_pager_slots_per_layer(const lp_pager* p);
/* Pager::request + wait_stream (pager.rs:402-460, 499-503): pin n experts of
 * `layer`; misses are copied from the host blobs on a copy stream; `compute`
 * waits for every fill still in flight and gets the layer's slot table
 * refreshed in its own order.  Never blocks for I/O; blocks only while every
 * slot of the pool is pinned and a release is pending; errors (expert cache
 * deadlock) when none is.  slots_out: n global slot numbers (may be NULL). */
int lp_pager_request(lp_pager* p, uint16_t layer, const uint16_t* experts, int n, lp_stream compute,
                     uint32_t* slots_out);
/* Pager::request (pager.rs:402-460): pin n experts of `layer` and schedule the
 * misses; returns at once with one handle per expert.  Before a kernel reads
 * handle i: lp_pager_wait_stream (or lp_pager_wait), and for the fused layer
 * kernels lp_pager_refresh_table. */
int lp_pager_request_handles(lp_pager* p, uint16_t layer, const uint16_t* experts, int n,
                             lp_expert_handle* out);
/* Pager::wait_stream (pager.rs:497-503): `s` waits for the handle's fill (the
 * host waits only until the copy is enqueued). */
int lp_pager_wait_stream(lp_pager* p, const lp_expert_handle* h, lp_stream s);
/* The layer's device slot table refreshed in stream order on `s` (no
 * counterpart in the reference, whose kernels take per-pick blob pointers). */
int lp_pager_refresh_table(lp_pager* p, uint16_t layer, lp_stream s);
/* Pager::release (pager.rs:505-510): unpin now (the GPU is done with them). */
int lp_pager_release(lp_pager* p, const uint32_t* slots, int n);
/* The deferred release of decode.rs:621-649: unpin once `compute` has passed
 * this point. */
int lp_pager_release_after(lp_pager* p, const uint32_t* slots, int n, lp_stream compute);
/* Pager::prefetch (pager.rs:464-486): best effort, never blocks; the fill's
 * pin drops when it lands. */
int lp_pager_prefetch(lp_pager* p, uint16_t layer, const uint16_t* experts, int n);
/* Pager::wait (pager.rs:489-496): block until the slot's last fill landed. */
int lp_pager_wait(lp_pager* p, uint32_t slot);
/* Pager::tick (pager.rs:524-533): end of a forward pass (global-pool decay). */
int lp_pager_tick(lp_pager* p);
/* Wait for every copy in flight and hand back every deferred release. */
int lp_pager_sync(lp_pager* p);
/* Pager::expert_stats (pager.rs:532-538): fills per (layer, expert), row-major;
 * copies min(n, layers * E) counts and returns layers * E. */
int lp_pager_expert_stats(lp_pager* p, uint64_t* counts, uint64_t n);
/* Pager::prewarm (pager.rs:540-567): the most-fetched experts of `counts`
 * that fit the RAM tier read into it, in pack order; returns how many (0
 * without a RAM tier). */
int lp_pager_prewarm(lp_pager* p, const uint64_t* counts, uint64_t n);
/* Pager::metrics (pager.rs:568-589). */
int lp_pager_get_metrics(lp_pager* p, lp_pager_metrics* out);

/* ---- the .llmpk pack (crates/llmpager-core/src/pack.rs) ------------------ */

typedef struct lp_pack lp_pack;
typedef struct lp_pack_writer lp_pack_writer;
/* PackWriter::create / add_blob / finish (pack.rs:67-150): blobs appended in
 * row-major (layer, expert) order, header and index written at finish. */
int lp_pack_create(const char* path, const char* model, const char* dtype, uint32_t layers, uint32_t experts,
                   lp_pack_writer** out);
int lp_pack_add_blob(lp_pack_writer* w, const void* blob, uint64_t nbytes);
int lp_pack_finish(lp_pack_writer* w);
/* PackReader::open / open_direct (pack.rs:152-205); compressed packs are
 * refused (LP_E_INVALID). */
int lp_pack_open(const char* path, int direct, lp_pack** out);
void lp_pack_close(lp_pack* p);
int lp_pack_info(const lp_pack* p, uint32_t* layers, uint32_t* experts, uint64_t* max_blob_bytes);
/* PackReader::entry (pack.rs:211-213) */
int lp_pack_entry(const lp_pack* p, uint32_t layer, uint32_t expert, uint64_t* offset, uint64_t* nbytes);
/* PackReader::read_blob_into (pack.rs:230-246): reads the blob's 4096-aligned
 * span (buf_len >= it; buf 4096-aligned under O_DIRECT); returns the blob's
 * length or a negative error. */
int64_t lp_pack_read_blob(lp_pack* p, uint32_t layer, uint32_t expert, void* buf, uint64_t buf_len);
/* pread of bytes [offset, offset + n) of the pack (4096-aligned under O_DIRECT). */
int lp_pack_read_range(lp_pack* p, uint64_t offset, void* buf, uint64_t n);

/* ---- measurement ------------------------------------------------------------ */

/* When enabled, every kernel launch through this context carries a start and
 * a stop hipEvent on its own dispatch (a measurement aid: the kernel's begin
 * and end timestamps, no separate event packets).  lp_profile_read_sync waits for the recorded work and
 * returns, for the kernel named `kernel` (e.g. "lp_moe_grouped"), the summed
 * elapsed milliseconds and launch count since the last reset. */
int lp_profile_enable(lp_ctx* ctx, int enable);
int lp_profile_reset(lp_ctx* ctx);
int lp_profile_read_sync(lp_ctx* ctx, const char* kernel, double* total_ms, int64_t* launches);

/* ---- blob format and synthetic inputs ------------------------------------ */

/* quant.rs:20-22 */
uint64_t lp_q4_bytes(int rows, int cols, int group);
/* Blob size (lib.rs:245-286) and the region offsets decode.rs:161-185 uses. */
uint64_t lp_blob_bytes(int hidden, int inter, int group);
void lp_blob_offsets(int hidden, int inter, int group, uint64_t* gate_off, uint64_t* up_off,
                     uint64_t* down_off);
/* Synthetic expert blob for (seed, layer, expert): header as lib.rs:276-281;
 * nibbles uniform 0..15; f16 scales round-to-nearest-even of |N(0, 0.02)|/8.
 * dst must hold lp_blob_bytes(). Deterministic, independent of threading. */
int lp_synth_blob(uint8_t* dst, int hidden, int inter, int group, uint64_t seed, int layer,
                  int expert);
/* n blobs (experts e0..e0+n-1 of `layer`), `stride` bytes apart, OpenMP-parallel. */
int lp_synth_blobs(uint8_t* dst, uint64_t stride, int n, int hidden, int inter, int group,
                   uint64_t seed, int layer, int e0, int threads);
/* bf16 bits of round-to-nearest-even N(0, std): router weights. */
int lp_synth_bf16(uint16_t* dst, uint64_t n, float std, uint64_t seed, uint64_t stream);
/* f32 values that are bf16-exact (RNE of N(0, std)): activations. */
int lp_synth_f32_bf16(float* dst, uint64_t n, float std, uint64_t seed, uint64_t stream);

/* Host evaluation of the expf routing uses (glibc's bits; see lp_expf.h). */
float lp_route_expf(float x);
/* out[i] = lp_route_expf(bits_to_float(first + i*stride)), i < n. */
void lp_route_expf_sweep(uint32_t first, uint32_t stride, uint64_t n, float* out);
/* The same sweep evaluated on the device the way the routing kernels do
 * (table in registers, whole waves); out: device f32 [n]. */
int lp_route_expf_device(lp_ctx* ctx, uint32_t first, uint32_t stride, uint64_t n, uint64_t out,
                         lp_stream s);

#ifdef __cplusplus
}
#endif

#endif /* LLMPAGER_HIP_H */
