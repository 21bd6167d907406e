// Kernel argument blocks shared by the host launchers (lp_runtime.cpp) and the
// gfx950 kernels (kernels/*.hip).  Every kernel takes exactly one of these by
// value, so hipModuleLaunchKernel is always given a single kernelParams entry
// and host/device layouts cannot drift apart.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define LPK_HD __host__ __device__
#else
#define LPK_HD
#endif

namespace lpk {

// Launch geometry constants the host and the kernels agree on.
constexpr int kWave = 64;              // CDNA wavefront
constexpr int kGroupedWaves = 4;       // waves per workgroup in the grouped kernels
constexpr int kTileRows = 16;          // weight rows per MFMA tile (N of 16x16x32)
constexpr int kRouterTokBlock = 8;     // tokens per router wave pass
constexpr int kRouteTokBlockMulti = 4;  // fused routing past one block: tokens per block (at most 16 blocks)
constexpr int kDispatchKeysMaxPicks = 64;  // a single token block of at most this many picks: dispatch by sort keys
constexpr int kRouteEPW = 1;           // fused routing: router experts per wave (8 waves per workgroup)
constexpr int kRouteXLds = 64 * 1024;  // fused routing: LDS for staged token rows (H <= 16384)
constexpr int kSyncSlots = 64;         // launch slots of the context's arrival counters
constexpr int kSyncStride = 32;        // words between arrival counters (one 128-byte line each)
// counters per slot: routing's [b] token block b (b < 16) and [16] every
// block, then the fused decode step's (kStepSyncAttn + g: attention's KV
// head g, kStepSyncGemv: the output projection)
constexpr int kAttnFusedMaxKvHeads = 16;
constexpr int kStepSyncAttn = 17 * kSyncStride;
constexpr int kStepSyncGemv = kStepSyncAttn + kAttnFusedMaxKvHeads * kSyncStride;
constexpr int kStepSyncDone = kStepSyncGemv + kSyncStride;  // lp_attn_block: KV heads complete
constexpr int kStepSyncErr = kStepSyncDone + kSyncStride;   // waits that gave up (lp_step_errors_sync)
constexpr int kSyncWords = kStepSyncErr + kSyncStride;
constexpr int kMaxTopK = 16;           // largest top_k the device router accepts
constexpr int kMaxExperts = 1024;      // largest expert count the device router accepts
constexpr int kTopkFusedMaxT = 8;      // largest T routed by the one-workgroup top-k + dispatch kernel
constexpr int kTopkDispatchMaxT = 64;  // largest T dispatched by one workgroup (after the top-k kernel)
constexpr int kDispTok = 256;          // tokens per block of the multi-block dispatch
constexpr int kMaxPairs = 2;           // token pairs the grouped kernels stage at once
constexpr int kMaxChunk = 16;          // most MFMA steps (4 sub-groups each) one register chunk holds
constexpr int kGateupChunk = 16;       // gate/up tiles up to this many steps load in one piece
constexpr int kGateupLoopChunk = 8;    // steps per chunk of longer gate/up tiles
constexpr int kDownChunk = 8;          // steps per chunk in the two-tile grouped down kernel
constexpr int kDownWideChunk = 16;     // one-tile down: tiles up to this many steps in one piece
constexpr int kDownLoopChunk = 8;      // steps per chunk of longer one-tile down tiles
constexpr int kGemvChunk = 8;          // steps per chunk in the 1:1 q4 GEMV
constexpr int kZeroBytes = 128 * kMaxChunk;  // LDS zero block read by idle MFMA lanes

// LDS bytes of the digit fragment area of the grouped q4 kernels for `pairs`
// token pairs over `cols` columns: a zero block, then per pair four
// (token, digit) blocks of ngp sub-groups x 32 B (+16 B to stagger banks),
// ngp x 16 B of accumulator seeds (int32: 0, seed of the pair's first token,
// 0, seed of its second) and ngp x 8 B of the two tokens' sub-group scales,
// with ngp = 4 * ceil(cols / 128) sub-groups (zero padded).
LPK_HD constexpr int frag_ngp(int cols) { return 4 * (((cols >> 5) + 3) >> 2); }
LPK_HD constexpr int frag_th_stride(int ngp) { return ngp * 32 + 16; }
LPK_HD constexpr int frag_off_bytes(int ngp) { return 4 * frag_th_stride(ngp); }
LPK_HD constexpr int frag_sig_bytes(int ngp) { return frag_off_bytes(ngp) + ngp * 16; }
LPK_HD constexpr int frag_pair_bytes(int ngp) { return frag_sig_bytes(ngp) + ngp * 8; }
LPK_HD constexpr int frag_lds_bytes(int cols, int pairs) {
    return kZeroBytes + pairs * frag_pair_bytes(frag_ngp(cols));
}

// A token row's digit image in device memory, the form the grouped q4
// kernels copy straight into LDS.  Each 32-column sub-group g is held as
// 16-bit fixed point against its own largest magnitude m: xq = rint(x *
// 32639 / m), split into digits hi = (xq + 128) >> 8 and lo = xq - 256 hi
// (both int8), with sigma = m / 32639; the blocks are hi [ngp][32 B] and lo
// [ngp][32 B] in MFMA operand order, then [ngp][2] int32 (0, -8 * sum xq)
// and sigma [ngp] f32.
LPK_HD constexpr int dimage_bytes(int cols) { return 76 * frag_ngp(cols); }
LPK_HD constexpr int dimage_seed_off(int ngp) { return 64 * ngp; }
LPK_HD constexpr int dimage_sigma_off(int ngp) { return 72 * ngp; }

// A token row's fp16 image, the token operand of the prefill GEMM: x * 2^-e
// rounded to fp16 (RNE) as [ngp][4][8] halves, where 16-byte word j of
// sub-group g holds columns 32 g + 8 j + (0, 4, 1, 5, 2, 6, 3, 7) (the order
// in which a q4 weight word unpacks), zero padding sub-groups past the last.
// The row's exponent e is kept beside it: x rows one per token (W.xexp, max
// |x| 2^-e in [2^14, 2^15)), act rows one per kActChunk columns (W.act).
LPK_HD constexpr int himage_bytes(int cols) { return 64 * frag_ngp(cols); }
constexpr int kActChunk = 128;       // act columns per exponent (one gate/up row block)
LPK_HD constexpr int act_chunks(int cols) { return frag_ngp(cols) >> 2; }
constexpr int kExpNone = -1024;      // exponent of an all-zero chunk

// The grouped kernels read a one-chunk tile's scales from a per-wave LDS
// window (filled by 16-byte copies of whole scale lines) when the group is 32
// and every row's scales start 16-byte aligned (sub-groups per row a
// multiple of 8); otherwise each lane loads its own.  The host adds the
// windows' bytes (scale_window_lds) to the launch's LDS.
LPK_HD constexpr bool scales_in_lds(int group, int cols) { return group == 32 && (cols >> 5) % 8 == 0; }
LPK_HD constexpr int scale_window_lds(int waves, int tiles_per_wave, int chunk_steps) {
    return waves * tiles_per_wave * 64 * 2 * chunk_steps;
}

// ---- 1:1 launchers (crates/llmpager-cuda/src/kernels.rs) -------------------

struct Q4GemvBatchArgs {            // kernels.rs:102-127
    uint64_t blobs;                 // device u64[experts] blob base addresses, or 0:
    uint64_t region_off;            //   then region_off is the region's device address
                                    //   (the single-matrix q4g64_gemv, kernels.rs:73-95)
    uint64_t x;                     // f32
    int32_t x_stride;
    int32_t pad0;
    uint64_t y;                     // f32 [experts, rows]
    int32_t rows, cols, group, experts;
};

struct MoeReduceArgs {              // kernels.rs:131-144
    uint64_t eouts, wts, out;
    int32_t experts, n;
};

struct SiluMulArgs {                // kernels.rs:224-236
    uint64_t gate, up, out;
    int32_t n, pad0;
};

struct Bf16GemvArgs {               // kernels.rs:202-222
    uint64_t w, x, y;
    int32_t rows, cols;
};

// The fused decode step (no reference counterpart: each fuses launches that
// decode.rs:275-301 issues one by one).
// y_i = W_i . rmsnorm(x, ln) (ln 0: W_i . x) for up to three bf16 [rows_i,
// cols] matrices sharing the input; cols a multiple of 8, at most
// kFusedGemvMaxCols.
constexpr int kFusedGemvMaxCols = 4096;
constexpr int kFusedGemvRowsPerWave = 2;  // rows per wave (4 waves per workgroup)
constexpr int kBlockRowsPerWave = 4;      // lp_attn_block's o projection
struct RmsNormGemvArgs {
    uint64_t x, ln;
    uint64_t w0, w1, w2, y0, y1, y2;
    int32_t rows0, rows1, rows2, cols;
    float eps;
    int32_t pad0;
};
// h[rows] += W . x (W bf16 [rows, cols]), then hn = rmsnorm(h, ln); rows at
// most kFusedGemvMaxRows
constexpr int kFusedGemvMaxRows = 4096;
struct GemvAddRmsNormArgs {
    uint64_t w, x, h, ln, hn, sync;
    int32_t rows, cols;
    float eps;
    int32_t pad0;
};
// Per-head q / k RMSNorm, NeoX RoPE, the fp16 KV append at pos and GQA
// decode attention over pos + 1 positions, head_dim 128; `cps` chunks of 64
// positions per split; partial records {acc[128], max, sum, 2 unused} at
// scratch + head * scratch_stride + split * kAttnFusedRec floats when
// splits > 1.
constexpr int kAttnFusedMaxSplits = 32;
constexpr int kAttnFusedRec = 128 + 4;
struct AttnFusedArgs {
    uint64_t q, k, v, q_norm, k_norm;
    uint64_t kcache, vcache, out, scratch, sync;
    int32_t kv_heads, pos, max_seq, splits, cps, scratch_stride;
    float eps, rope_base, scale;
    int32_t pad0;
};

// lp_attn_fused on workgroups [0, n_attn) (at.out the attention output),
// then h[rows] += W_o . out (W_o bf16 [rows, cols]) and hn = rmsnorm(h, ln)
// on the workgroups after them
constexpr int kStepSpinMax = 1 << 15;  // polls (about a microsecond each) before the wait gives up
struct AttnBlockArgs {
    AttnFusedArgs at;
    uint64_t wo, h, ln, hn;
    int32_t rows, cols, n_attn, spin_max;
};

struct AddArgs {                    // kernels.rs:239-250
    uint64_t a, b;
    int32_t n, pad0;
};

struct ExpfSweepArgs {              // device expf check (no reference counterpart)
    uint64_t out;                   // f32 [n]
    uint64_t n;
    uint32_t first, stride;
};

// ---- the rest of the decode step (decode.cu) and MLA (mla.cu) ----------------

struct RmsNormArgs {                // kernels.rs:145-158 (rmsnorm_f32); rows = grid
    uint64_t x, w, y;
    int32_t n;
    float eps;
};

struct ScaleAddArgs {               // kernels.rs:161-173 (scale_add_f32)
    uint64_t a, b;
    float s;
    int32_t n;
};

struct KvAppendArgs {               // kernels.rs:176-196 (kv_append_f32 / _f16)
    uint64_t k, v, kcache, vcache;
    int32_t kv_heads, head_dim, pos, max_seq;
};

struct RopeArgs {                   // kernels.rs:252-266 (rope_f32, NeoX rotate-half)
    uint64_t x;
    int32_t heads, head_dim, pos;
    float base;
};

struct RowArgs {                    // kernels.rs:294-306 (bf16_row_to_f32)
    uint64_t table, out;
    int32_t row, n;
};

struct MlaRopeArgs {                // kernels.rs:311-330 (mla_rope_f32, interleaved pairs)
    uint64_t x, inv_freq;
    int32_t n_vecs, stride, offset, half, pos;
    float mscale;
};

struct Bf16GemvBatchArgs {          // kernels.rs:357-381 (bf16_gemv_batch)
    uint64_t w, w_stride, x, y;     // w_stride in elements
    int32_t x_stride, y_stride, rows, cols, batch, pad0;
};

struct StridedCopyArgs {            // kernels.rs:386-404 (strided_copy_f32)
    uint64_t src, dst;
    int32_t src_stride, src_off, dst_stride, dst_off, n_vecs, n;
};

// Decode attention over one query per head (attn_decode_f32 / _f16kv,
// kernels.rs:269-292; mla_attn_decode_f32, kernels.rs:333-354), split over
// positions: split s of head h covers positions [s span, (s + 1) span) and
// either writes the head's output (one split) or a partial record
// {max, sum, acc[out_dim]} at scratch + h * scratch_stride + s * (out_dim + 2)
// that lp_attn_combine merges.  Keys of head h: k + (h / group) * kv_stride,
// row p at p * row_stride elements, `dot_dim` wide; values likewise from v,
// `out_dim` wide.  GQA decode has k != v; MLA reads both from its one cache.
constexpr int kAttnSpanMax = 1024;  // positions per split (LDS scores)
struct AttnArgs {
    uint64_t q, k, v, out, scratch;
    uint64_t kv_stride;             // elements between kv heads' caches
    int32_t heads, group;           // query heads, query heads per kv head
    int32_t dot_dim, out_dim, row_stride, seq_len;
    int32_t splits, span, scratch_stride;
    float scale;
    int32_t f16;                    // caches hold IEEE half (else f32)
    int32_t pad0;
};

// The batched MLA decode of config 5 (no reference counterpart: the
// reference runs mla_attn_decode_f32 once per sequence over an f32 cache):
// bf16 latent caches, MFMA scores and context, splits of `span` positions
// (a multiple of kMlaRows) per workgroup, partial records merged by
// lp_mla_combine.  Heads <= 16, qk_dim a multiple of 32 (<= kMlaMaxQk),
// c_dim a multiple of 64 (<= kMlaMaxC).
constexpr int kMlaRows = 64;        // cache rows per chunk (4 waves x 16)
constexpr int kMlaMaxQk = 640;
constexpr int kMlaMaxC = 512;
constexpr int kMlaMaxSplits = 256;  // splits per sequence (the merge keeps one weight per split in LDS)
// Bytes per row of the chunk staged in LDS: c_dim bf16 and 32 bytes of pad,
// so that the four rows one 16-lane group of a transposing read touches
// start 8 banks apart.
LPK_HD constexpr int mla_row_bytes(int c_dim) { return 2 * c_dim + 32; }
// LDS: the query images (hi and lo bf16 in MFMA A order, 2 x qk/32 x 1 KB),
// the chunk's rows (kMlaRows x mla_row_bytes) and the scores (16 x 64 f32).
LPK_HD constexpr int mla_lds_bytes(int qk_dim, int c_dim) {
    return 2 * (qk_dim / 32) * 1024 + kMlaRows * mla_row_bytes(c_dim) + 16 * kMlaRows * 4;
}
// Floats of one partial record: max[16], sum[16], acc[16][c_dim].
LPK_HD constexpr int mla_part_floats(int c_dim) { return 32 + 16 * c_dim; }
struct MlaBatchArgs {
    uint64_t q;                     // f32 [batch][heads][qk_dim]
    uint64_t cache;                 // bf16; sequence b's rows at cache + b * cache_stride bytes
    uint64_t cache_stride;          // bytes
    uint64_t seq_lens;              // i32 [batch]
    uint64_t ctx;                   // f32 [batch][heads][c_dim]
    uint64_t part;                  // f32 [batch][splits] partial records
    int32_t batch, heads, qk_dim, c_dim, splits, span;
    float scale;
    int32_t max_seq;                // rows per cache: seq_lens[b] is clamped to it on the device
};

// ---- fused MoE layer ---------------------------------------------------------

// Device-side view of one MoE layer's routing and expert tables.
struct LayerView {
    uint64_t router_w;       // bf16 [E, H]
    uint64_t router_bias;    // f32 [E] or 0
    uint64_t slot_table;     // int32 [E]: slot within the arena, -1 = absent
    uint64_t arena_base;     // device base of the layer's slot arena
    uint64_t slot_span;      // bytes per slot
    uint64_t gate_off, up_off, down_off;
    int32_t hidden, inter, experts, top_k, group;
    int32_t gating;          // 0 softmax, 1 sigmoid + bias
    int32_t renorm;
    float routed_scaling, min_weight;
    int32_t pad0;
    uint64_t shared_blob;    // the always-on shared MLP's blob, or 0
    uint64_t sh_gate_off, sh_up_off, sh_down_off;
    int32_t shared_inter, shared_group;
};

// One routed expert as the grouped kernels see it, written by the dispatch
// kernel for u < min(T*k, E) (ntok = 0 past the unique count).
constexpr int kEntryToks = 4;  // tokens an entry names directly (2 * kMaxPairs)
struct ExpertEntry {
    uint64_t blob;             // device address of the expert's blob (0 if not resident)
    int32_t p0;                // first dispatch position of its (token, pick) pairs
    int32_t ntok;              // number of those pairs
    int32_t tok[kEntryToks];   // tokens of the first pairs (-1 if absent)
};
static_assert(sizeof(ExpertEntry) == 32, "two 16-byte loads per entry");
static_assert(2 * kMaxPairs <= kEntryToks, "the first token group comes from the entry");

// Workspace carve-up for T tokens (offsets in bytes from `ws`).
struct Workspace {
    uint64_t logits;     // f32 [T, E]
    uint64_t ids;        // i32 [T, k]
    uint64_t wts;        // f32 [T, k]
    uint64_t cnt;        // i32 [T]
    uint64_t gs;         // i32 [E + 1] group starts
    uint64_t perm;       // i32 [T * k] pick (t*k+j) per dispatch position
    uint64_t inv;        // i32 [T * k] dispatch position per pick (-1 if none)
    uint64_t uniq;       // i32 [E] experts with picks, ascending
    uint64_t meta;       // i32 [16]: [0] = unique count, [1] = error flags
    uint64_t et;         // ExpertEntry [E]
    uint64_t act;        // f32 [T * k, I] expert-major activations; prefill GEMM: i32 [T * k][act_chunks(I)] act image exponents
    uint64_t y;          // f32 [T * k, H] expert-major expert outputs
    uint64_t xf;         // [T] fp16 images of the layer input for the prefill GEMM (himage_bytes(H) each)
    uint64_t xd;         // [T] digit images of the layer input for the grouped kernels (dimage_bytes(H) each)
    uint64_t sh_et;      // shared MLP: shared_entries(T) ExpertEntry (consecutive tokens)
    uint64_t sh_perm;    // shared MLP: i32 [T], t
    uint64_t sh_act;     // shared MLP: f32 [T, shared_inter]
    uint64_t sh_y;       // shared MLP: f32 [T, H]
    uint64_t tiles;      // prefill GEMM: i32 tile list
    uint64_t actimg;     // prefill GEMM: [T*k] fp16 images of act rows (himage_bytes(I) each)
    uint64_t xexp;       // prefill GEMM: i32 [T], token t's image exponent in xf
    uint64_t disp;       // multi-block dispatch: i32 [nb][E] counts, [nb][E] first positions, [E] entries
};

// Entries of the shared MLP's expert table: groups of kEntryToks consecutive
// tokens for decode batches (the grouped kernels then need no token loop),
// one entry of all T tokens above 64.
LPK_HD constexpr int shared_entries(int T) { return T <= 64 ? (T + kEntryToks - 1) / kEntryToks : 1; }

constexpr int kImgF16 = 1;     // RouteArgs::make_xf bits
constexpr int kImgDigits = 2;

struct RouteArgs {
    LayerView L;
    Workspace W;
    uint64_t x;          // f32 [T, H]
    int32_t T;
    int32_t make_xf;     // router: also write images of x: kImgF16 into W.xf (+ W.xexp), kImgDigits into W.xd
    uint64_t sync;       // fused routing: kSyncWords arrival counters, zero between launches
    int32_t tok_block;   // fused routing: tokens per block (grid y = ceil(T / tok_block))
    int32_t pad0;
};

struct GroupedArgs {
    LayerView L;
    Workspace W;
    uint64_t x;          // f32 [T, H] (gate/up phase input)
    uint64_t h;          // f32 [T, H] residual (combine)
    int32_t T;
    int32_t pairs_cap;   // token pairs the dynamic LDS holds at once
    int32_t maxu;        // expert-table entries (balanced kernels)
    int32_t sh_fused;    // lp_moe_down_comb_rs: also the shared MLP's down (its act row in W.sh_act)
    int32_t sh_maxu;     // balanced gate/up: the shared MLP's W.sh_et entries taken after the routed ones
    int32_t wave_u0;     // combine of one wave (wave_n > 0): the routed experts uniq[wave_u0 ..
    int32_t wave_n;      //   wave_u0 + wave_n) only; tokens without a pick among them are left as they are
    int32_t pad0;
};

// Balanced decode gate/up (lp_moe_gateup_bal): one workgroup of kBalWaves
// waves per CU (the kernels' launch bound; the only size they are built and
// tested for).  LDS: the zero block and two slots of kBalGroups * kBalPairs
// token pairs (frag_lds_bytes(H, 2 kBalGroups kBalPairs)), 128 bytes of
// counters (kBalWaves wave totals, then six slot words), the expert table
// (kBalMaxU entries), then one scale window per wave.
constexpr int kBalWaves = 8;
// A token group of the balanced kernels: up to kBalPairs token pairs of one
// routed expert, which one unit's MFMAs serve.  Groups of four pairs were
// measured slower at 32 tokens: the units of one range then differ up to
// fourfold in MFMA work (the row-major blocks below save the weight bytes
// instead).
constexpr int kBalPairs = 2;
constexpr int kBalToks = 2 * kBalPairs;
// Token groups of one expert whose units the balanced kernels interleave
// (neighbouring units read the same weight rows for different groups).
constexpr int kBalGroups = 2;
constexpr int kBalMaxU = 64 * kBalWaves;
// Row tiles (16 rows of down, all of K) in one unit of the balanced down.
// Two (12 KB of nibbles per unit at inter 768, half the units) measured
// slower: 26.3 against 25.1 us at 32 tokens.
constexpr int kDownBalTiles = 1;
static_assert(4 * kBalWaves + 24 <= 128, "bal_plan's counters fit their 128 bytes");
LPK_HD constexpr int bal_meta_off(int hidden) {
    return (frag_lds_bytes(hidden, 2 * kBalGroups * kBalPairs) + 15) & ~15;
}
LPK_HD constexpr int bal_win_off(int hidden) { return bal_meta_off(hidden) + 128 + kBalMaxU * 32; }
LPK_HD constexpr int bal_lds_bytes(int hidden, int window_steps, int waves) {
    return bal_win_off(hidden) + waves * 64 * 2 * window_steps;
}

// One-token down + combine (lp_moe_down_comb): one wave per pick; with the
// shared MLP's down fused in, its two halves of K on the last two waves.
constexpr int kCombWaves = 8;
constexpr int kCombShWaves = 2;

// Prefill grouped GEMM (lp_gemm.hip).  A tile is 128 tokens x 256 weight
// rows (gate/up: 128 act columns, their gate and up rows), kGemmWaves waves of
// kGemmRowTiles 16-row MFMA tiles; K runs in stages of 64 columns.
constexpr int kGemmBM = 128;           // tokens per tile
constexpr int kGemmBN = 256;           // weight rows per tile
constexpr int kGemmRowTiles = 2;      // 16-row MFMA tiles per wave
constexpr int kGemmWaves = kGemmBN / (16 * kGemmRowTiles);
constexpr int kGemmMinPairsPerExpert = 16;  // the experts path switches to the GEMM at this average
constexpr int kXcds = 8;               // MI355X: workgroup w is dispatched to XCD w % 8
constexpr int kGemmMaxChunks = 64;     // act chunks per row the down GEMM's LDS table holds (I <= 8192)

// GEMM LDS.  Token rows (128 B of each of the 128 tokens per stage) and weight
// rows (32 B of each of the 256 rows per stage) in four slots each, loads
// three stages ahead; scale windows (16 f16 of each row, every 4 stages) in
// two; then the tile's row table, exponents and the down GEMM's per-(token,
// chunk) exponent shifts.
constexpr int kGemmSlots = 4;
constexpr int kGemmSlotT = kGemmBM * 128;                      // 16 KiB
constexpr int kGemmSlotW = kGemmBN * 32;                       // 8 KiB
constexpr int kGemmSlotS = kGemmBN * 32;                       // 8 KiB
constexpr int kGemmLdsW = kGemmSlots * kGemmSlotT;             // 65,536
constexpr int kGemmLdsS = kGemmLdsW + kGemmSlots * kGemmSlotW; // 98,304
constexpr int kGemmLdsRows = kGemmLdsS + 2 * kGemmSlotS;       // 114,688: u32 image offset per tile row
constexpr int kGemmLdsExp = kGemmLdsRows + kGemmBM * 4;        // i32 exponent per tile row
constexpr int kGemmLdsShift = kGemmLdsExp + kGemmBM * 4;       // i8 [128][kGemmMaxChunks]
constexpr int kGemmLds = kGemmLdsShift + kGemmBM * kGemmMaxChunks;  // 123,904

struct GemmArgs {
    LayerView L;
    Workspace W;
    uint64_t a_img;      // token images: gate/up = W.xf (token rows through perm); down = W.actimg
    uint64_t out;        // gate/up: act images [T*k] (himage_bytes(I) each); down: y f32 [T*k, H]
    uint64_t tiles;      // i32 [max_tiles]: (expert entry << 16) | token block; count in meta[2]
    int32_t T;
    int32_t max_tiles;
    int32_t nblocks;     // weight-row blocks per tile row
    int32_t pad0;
};

// Error flags written into Workspace.meta[1].
constexpr int kErrMissingExpert = 1;  // a routed expert had no slot
constexpr int kErrBadShape = 2;

}  // namespace lpk
