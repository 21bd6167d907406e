//! Raw declarations of the C ABI in `include/llmpager_hip.h`.  The header is
//! the authority; every declaration there cites the reference method it
//! replaces.  Device pointers are `u64`, as `CUdeviceptr` is in
//! `llmpager-cuda/src/driver.rs`.
#![allow(non_camel_case_types, dead_code)]

use std::os::raw::{c_char, c_int, c_void};

#[repr(C)]
pub struct lp_ctx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct lp_pager {
    _p: [u8; 0],
}
#[repr(C)]
pub struct lp_cache {
    _p: [u8; 0],
}
#[repr(C)]
pub struct lp_graph {
    _p: [u8; 0],
}
#[repr(C)]
pub struct lp_pack {
    _p: [u8; 0],
}
#[repr(C)]
pub struct lp_pack_writer {
    _p: [u8; 0],
}

pub type lp_stream = *mut c_void;
pub type lp_event = *mut c_void;

pub const LP_OK: c_int = 0;
pub const LP_E_INVALID: c_int = -1;
pub const LP_E_UNSUPPORTED: c_int = -2;
pub const LP_E_LOAD: c_int = -3;
pub const LP_E_DEVICE: c_int = -5;

pub const LP_GATING_SOFTMAX: i32 = 0;
pub const LP_GATING_SIGMOID: i32 = 1;

pub const LP_LOOKUP_HIT: c_int = 0;
pub const LP_LOOKUP_MISS: c_int = 1;
pub const LP_LOOKUP_STALLED: c_int = 2;

pub const LP_PAGER_SRC_PINNED: i32 = 0;
pub const LP_PAGER_SRC_HOST: i32 = 1;
pub const LP_PAGER_SRC_PACK: i32 = 2;

pub const LP_NOALLOC_SCRATCH_BYTES: u64 = 16 << 20;

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct lp_moe_layer_desc {
    pub hidden: i32,
    pub inter: i32,
    pub experts: i32,
    pub top_k: i32,
    pub group: i32,
    pub gating: i32,
    pub renorm: i32,
    pub routed_scaling: f32,
    pub min_weight: f32,
    pub reserved0: i32,
    pub router_w: u64,
    pub router_bias: u64,
    pub slot_table: u64,
    pub arena_base: u64,
    pub slot_span: u64,
    pub gate_off: u64,
    pub up_off: u64,
    pub down_off: u64,
    pub shared_blob: u64,
    pub shared_inter: i32,
    pub shared_group: i32,
    pub sh_gate_off: u64,
    pub sh_up_off: u64,
    pub sh_down_off: u64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct lp_moe_ws_layout {
    pub logits: u64,
    pub ids: u64,
    pub wts: u64,
    pub cnt: u64,
    pub gs: u64,
    pub perm: u64,
    pub inv: u64,
    pub uniq: u64,
    pub meta: u64,
    pub et: u64,
    pub act: u64,
    pub y: u64,
    pub xf: u64,
    pub xd: u64,
    pub sh_et: u64,
    pub sh_perm: u64,
    pub sh_act: u64,
    pub sh_y: u64,
    pub tiles: u64,
    pub actimg: u64,
    pub xexp: u64,
    pub disp: u64,
    pub total: u64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct lp_pager_config {
    pub layers: u32,
    pub experts_per_layer: u32,
    pub slots_per_layer: u32,
    pub decay_interval: u32,
    pub blob_bytes: u64,
    pub span: u64,
    pub host_blobs: *const c_void,
    pub host_stride: u64,
    pub copy_streams: i32,
    pub global_pool: i32,
    pub pool_decay_tokens: u32,
    pub source: i32,
    pub direct: i32,
    pub io_threads: u32,
    pub ring_slots: u32,
    pub stage_threads: u32,
    pub ram_bytes: u64,
    pub reserve_bytes: u64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct lp_pager_metrics {
    pub hits: u64,
    pub misses: u64,
    pub bytes_fetched: u64,
    pub fetches: u64,
    pub stalls: u64,
    pub ram_hits: u64,
    pub latency_ms_buckets: [u64; 7],
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct lp_expert_handle {
    pub layer: u16,
    pub expert: u16,
    pub slot: u32,
    pub dev: u64,
    pub len: u64,
}

extern "C" {
    pub fn lp_last_error() -> *const c_char;
    pub fn lp_version() -> *const c_char;

    // ---- device runtime: driver::Cuda ----
    pub fn lp_init(device: c_int, hsaco_dir: *const c_char, out: *mut *mut lp_ctx) -> c_int;
    pub fn lp_destroy(ctx: *mut lp_ctx);
    pub fn lp_bind_thread(ctx: *mut lp_ctx) -> c_int;
    pub fn lp_mem_info(ctx: *mut lp_ctx, free_bytes: *mut u64, total_bytes: *mut u64) -> c_int;
    pub fn lp_alloc_device(ctx: *mut lp_ctx, bytes: usize, out: *mut u64) -> c_int;
    pub fn lp_free_device(ctx: *mut lp_ctx, ptr: u64) -> c_int;
    pub fn lp_alloc_pinned(ctx: *mut lp_ctx, bytes: usize, out: *mut *mut c_void) -> c_int;
    pub fn lp_free_pinned(ctx: *mut lp_ctx, p: *mut c_void) -> c_int;
    pub fn lp_stream_create(ctx: *mut lp_ctx, out: *mut lp_stream) -> c_int;
    pub fn lp_stream_destroy(ctx: *mut lp_ctx, s: lp_stream) -> c_int;
    pub fn lp_event_create(ctx: *mut lp_ctx, out: *mut lp_event) -> c_int;
    pub fn lp_event_destroy(ctx: *mut lp_ctx, e: lp_event) -> c_int;
    pub fn lp_htod_async(ctx: *mut lp_ctx, dst: u64, src: *const c_void, bytes: usize, s: lp_stream) -> c_int;
    pub fn lp_dtoh_async(ctx: *mut lp_ctx, dst: *mut c_void, src: u64, bytes: usize, s: lp_stream) -> c_int;
    pub fn lp_dtod_async(ctx: *mut lp_ctx, dst: u64, src: u64, bytes: usize, s: lp_stream) -> c_int;
    pub fn lp_memset_async(ctx: *mut lp_ctx, dst: u64, value: c_int, bytes: usize, s: lp_stream) -> c_int;
    pub fn lp_record_event(ctx: *mut lp_ctx, e: lp_event, s: lp_stream) -> c_int;
    pub fn lp_sync_event(ctx: *mut lp_ctx, e: lp_event) -> c_int;
    pub fn lp_event_done(ctx: *mut lp_ctx, e: lp_event) -> c_int;
    pub fn lp_event_elapsed_ms(ctx: *mut lp_ctx, start: lp_event, end: lp_event, ms: *mut f32) -> c_int;
    pub fn lp_stream_wait_event(ctx: *mut lp_ctx, s: lp_stream, e: lp_event) -> c_int;
    pub fn lp_sync_stream(ctx: *mut lp_ctx, s: lp_stream) -> c_int;
    pub fn lp_sync(ctx: *mut lp_ctx) -> c_int;

    // ---- hot-path launchers: kernels::Kernels ----
    pub fn lp_q4_gemv_batch(
        ctx: *mut lp_ctx, blobs: u64, region_off: u64, x: u64, x_stride: c_int, y: u64, rows: c_int,
        cols: c_int, group: c_int, experts: c_int, s: lp_stream,
    ) -> c_int;
    pub fn lp_q4_gemv(
        ctx: *mut lp_ctx, blob: u64, x: u64, y: u64, rows: c_int, cols: c_int, group: c_int, s: lp_stream,
    ) -> c_int;
    pub fn lp_moe_reduce(
        ctx: *mut lp_ctx, eouts: u64, wts: u64, out: u64, experts: c_int, n: c_int, s: lp_stream,
    ) -> c_int;
    pub fn lp_silu_mul(ctx: *mut lp_ctx, gate: u64, up: u64, out: u64, n: c_int, s: lp_stream) -> c_int;
    pub fn lp_bf16_gemv(ctx: *mut lp_ctx, w: u64, x: u64, y: u64, rows: c_int, cols: c_int, s: lp_stream) -> c_int;
    pub fn lp_add(ctx: *mut lp_ctx, a: u64, b: u64, n: c_int, s: lp_stream) -> c_int;
    pub fn lp_rmsnorm(
        ctx: *mut lp_ctx, x: u64, w: u64, y: u64, rows: c_int, n: c_int, eps: f32, s: lp_stream,
    ) -> c_int;
    pub fn lp_scale_add(ctx: *mut lp_ctx, a: u64, b: u64, s_: f32, n: c_int, s: lp_stream) -> c_int;
    pub fn lp_kv_append(
        ctx: *mut lp_ctx, k: u64, v: u64, kcache: u64, vcache: u64, kv_heads: c_int, head_dim: c_int,
        pos: c_int, max_seq: c_int, f16: c_int, s: lp_stream,
    ) -> c_int;
    pub fn lp_rope(
        ctx: *mut lp_ctx, x: u64, heads: c_int, head_dim: c_int, pos: c_int, base: f32, s: lp_stream,
    ) -> c_int;
    pub fn lp_attn_decode(
        ctx: *mut lp_ctx, q: u64, kcache: u64, vcache: u64, out: u64, scratch: u64, heads: c_int,
        kv_heads: c_int, head_dim: c_int, seq_len: c_int, max_seq: c_int, scale: f32, f16: c_int, s: lp_stream,
    ) -> c_int;
    pub fn lp_bf16_row(ctx: *mut lp_ctx, table: u64, row: c_int, n: c_int, out: u64, s: lp_stream) -> c_int;
    pub fn lp_rmsnorm_gemv(
        ctx: *mut lp_ctx, x: u64, ln: u64, eps: f32, cols: c_int, w0: u64, rows0: c_int, y0: u64, w1: u64,
        rows1: c_int, y1: u64, w2: u64, rows2: c_int, y2: u64, s: lp_stream,
    ) -> c_int;
    pub fn lp_gemv_add_rmsnorm(
        ctx: *mut lp_ctx, w: u64, x: u64, rows: c_int, cols: c_int, h: u64, ln: u64, eps: f32, hn: u64,
        s: lp_stream,
    ) -> c_int;
    pub fn lp_attn_fused(
        ctx: *mut lp_ctx, q: u64, k: u64, v: u64, q_norm: u64, k_norm: u64, eps: f32, rope_base: f32,
        kcache: u64, vcache: u64, out: u64, scratch: u64, heads: c_int, kv_heads: c_int, head_dim: c_int,
        pos: c_int, max_seq: c_int, scale: f32, s: lp_stream,
    ) -> c_int;
    pub fn lp_attn_block(
        ctx: *mut lp_ctx, q: u64, k: u64, v: u64, q_norm: u64, k_norm: u64, eps: f32, rope_base: f32,
        kcache: u64, vcache: u64, att: u64, scratch: u64, heads: c_int, kv_heads: c_int, head_dim: c_int,
        pos: c_int, max_seq: c_int, scale: f32, wo: u64, h: u64, post_ln: u64, hn: u64, hidden: c_int,
        s: lp_stream,
    ) -> c_int;
    pub fn lp_step_errors_sync(ctx: *mut lp_ctx, timeouts: *mut i32) -> c_int;
    pub fn lp_mla_rope(
        ctx: *mut lp_ctx, x: u64, n_vecs: c_int, stride: c_int, offset: c_int, half: c_int, pos: c_int,
        inv_freq: u64, mscale: f32, s: lp_stream,
    ) -> c_int;
    pub fn lp_mla_attn_decode(
        ctx: *mut lp_ctx, q: u64, cache: u64, ctx_out: u64, scratch: u64, heads: c_int, qk_dim: c_int,
        c_dim: c_int, seq_len: c_int, max_seq: c_int, scale: f32, s: lp_stream,
    ) -> c_int;
    pub fn lp_bf16_gemv_batch(
        ctx: *mut lp_ctx, w: u64, w_stride: u64, x: u64, x_stride: c_int, y: u64, y_stride: c_int, rows: c_int,
        cols: c_int, batch: c_int, s: lp_stream,
    ) -> c_int;
    pub fn lp_strided_copy(
        ctx: *mut lp_ctx, src: u64, src_stride: c_int, src_off: c_int, dst: u64, dst_stride: c_int,
        dst_off: c_int, n_vecs: c_int, n: c_int, s: lp_stream,
    ) -> c_int;
    pub fn lp_mla_batch_ws_bytes(ctx: *mut lp_ctx, batch: c_int, c_dim: c_int, max_seq: c_int) -> u64;
    pub fn lp_mla_attn_decode_batch(
        ctx: *mut lp_ctx, q: u64, cache: u64, cache_stride: u64, seq_lens: u64, ctx_out: u64, workspace: u64,
        batch: c_int, heads: c_int, qk_dim: c_int, c_dim: c_int, max_seq: c_int, scale: f32, s: lp_stream,
    ) -> c_int;

    // ---- the fused MoE layer ----
    pub fn lp_moe_ws_layout_get(d: *const lp_moe_layer_desc, t: c_int, out: *mut lp_moe_ws_layout) -> c_int;
    pub fn lp_moe_workspace_check(
        layers: *const lp_moe_layer_desc, n_layers: c_int, t: c_int, workspace: u64, ws_bytes: u64,
    ) -> c_int;
    pub fn lp_moe_route(
        ctx: *mut lp_ctx, d: *const lp_moe_layer_desc, x: u64, t: c_int, ws: u64, ws_bytes: u64, s: lp_stream,
    ) -> c_int;
    pub fn lp_moe_route_logits(
        ctx: *mut lp_ctx, d: *const lp_moe_layer_desc, logits: u64, t: c_int, ws: u64, ws_bytes: u64, s: lp_stream,
    ) -> c_int;
    pub fn lp_moe_experts(
        ctx: *mut lp_ctx, d: *const lp_moe_layer_desc, x: u64, h: u64, t: c_int, ws: u64, ws_bytes: u64,
        s: lp_stream,
    ) -> c_int;
    pub fn lp_moe_experts_wave(
        ctx: *mut lp_ctx, d: *const lp_moe_layer_desc, x: u64, h: u64, t: c_int, ws: u64, ws_bytes: u64,
        u_first: c_int, u_count: c_int, with_shared: c_int, s: lp_stream,
    ) -> c_int;
    pub fn lp_moe_resolve(
        ctx: *mut lp_ctx, d: *const lp_moe_layer_desc, t: c_int, ws: u64, ws_bytes: u64, s: lp_stream,
    ) -> c_int;
    pub fn lp_moe_forward(
        ctx: *mut lp_ctx, d: *const lp_moe_layer_desc, x: u64, h: u64, t: c_int, ws: u64, ws_bytes: u64,
        s: lp_stream,
    ) -> c_int;
    pub fn lp_moe_stack_forward(
        ctx: *mut lp_ctx, layers: *const lp_moe_layer_desc, n_layers: c_int, h: u64, t: c_int, ws: u64,
        ws_bytes: u64, s: lp_stream,
    ) -> c_int;
    pub fn lp_moe_stack_capture(
        ctx: *mut lp_ctx, layers: *const lp_moe_layer_desc, n_layers: c_int, h: u64, t: c_int, ws: u64,
        ws_bytes: u64, s: lp_stream, out: *mut *mut lp_graph,
    ) -> c_int;
    pub fn lp_graph_capture_begin(ctx: *mut lp_ctx, s: lp_stream) -> c_int;
    pub fn lp_graph_capture_end(ctx: *mut lp_ctx, s: lp_stream, out: *mut *mut lp_graph) -> c_int;
    pub fn lp_graph_launch(ctx: *mut lp_ctx, g: *mut lp_graph, s: lp_stream) -> c_int;
    pub fn lp_graph_destroy(g: *mut lp_graph);
    pub fn lp_moe_forward_noalloc(
        ctx: *mut lp_ctx, d: *const lp_moe_layer_desc, x: u64, h: u64, t: c_int, s: lp_stream,
    ) -> c_int;
    pub fn lp_noalloc_scratch_bytes() -> u64;
    pub fn lp_moe_status_sync(
        ctx: *mut lp_ctx, ws: u64, ws_bytes: u64, d: *const lp_moe_layer_desc, t: c_int, s: lp_stream,
        unique_count: *mut i32, error_flags: *mut i32,
    ) -> c_int;

    // ---- expert-slot bookkeeping: cache::ExpertCache ----
    pub fn lp_cache_new(num_layers: u16, slots_per_layer: u32, decay_interval: u32) -> *mut lp_cache;
    pub fn lp_cache_free(c: *mut lp_cache);
    pub fn lp_cache_acquire(c: *mut lp_cache, id: u32, slot: *mut u32, evicted: *mut i64) -> c_int;
    pub fn lp_cache_publish(c: *mut lp_cache, slot: u32) -> c_int;
    pub fn lp_cache_release(c: *mut lp_cache, slot: u32) -> c_int;

    // ---- expert pager: pager::Pager ----
    pub fn lp_pager_new(ctx: *mut lp_ctx, cfg: *const lp_pager_config, out: *mut *mut lp_pager) -> c_int;
    pub fn lp_pager_open(
        ctx: *mut lp_ctx, pack_path: *const c_char, cfg: *const lp_pager_config, out: *mut *mut lp_pager,
    ) -> c_int;
    pub fn lp_pager_free(p: *mut lp_pager);
    pub fn lp_pager_arena(p: *const lp_pager) -> u64;
    pub fn lp_pager_span(p: *const lp_pager) -> u64;
    pub fn lp_pager_slot_table(p: *const lp_pager, layer: u32) -> u64;
    pub fn lp_pager_slots_per_layer(p: *const lp_pager) -> u32;
    pub fn lp_pager_request(
        p: *mut lp_pager, layer: u16, experts: *const u16, n: c_int, compute: lp_stream, slots_out: *mut u32,
    ) -> c_int;
    pub fn lp_pager_request_handles(
        p: *mut lp_pager, layer: u16, experts: *const u16, n: c_int, out: *mut lp_expert_handle,
    ) -> c_int;
    pub fn lp_pager_wait_stream(p: *mut lp_pager, h: *const lp_expert_handle, s: lp_stream) -> c_int;
    pub fn lp_pager_refresh_table(p: *mut lp_pager, layer: u16, s: lp_stream) -> c_int;
    pub fn lp_pager_release(p: *mut lp_pager, slots: *const u32, n: c_int) -> c_int;
    pub fn lp_pager_release_after(p: *mut lp_pager, slots: *const u32, n: c_int, compute: lp_stream) -> c_int;
    pub fn lp_pager_prefetch(p: *mut lp_pager, layer: u16, experts: *const u16, n: c_int) -> c_int;
    pub fn lp_pager_wait(p: *mut lp_pager, slot: u32) -> c_int;
    pub fn lp_pager_tick(p: *mut lp_pager) -> c_int;
    pub fn lp_pager_sync(p: *mut lp_pager) -> c_int;
    pub fn lp_pager_expert_stats(p: *mut lp_pager, counts: *mut u64, n: u64) -> c_int;
    pub fn lp_pager_prewarm(p: *mut lp_pager, counts: *const u64, n: u64) -> c_int;
    pub fn lp_pager_get_metrics(p: *mut lp_pager, out: *mut lp_pager_metrics) -> c_int;

    // ---- the .llmpk pack ----
    pub fn lp_pack_create(
        path: *const c_char, model: *const c_char, dtype: *const c_char, layers: u32, experts: u32,
        out: *mut *mut lp_pack_writer,
    ) -> c_int;
    pub fn lp_pack_add_blob(w: *mut lp_pack_writer, blob: *const c_void, nbytes: u64) -> c_int;
    pub fn lp_pack_finish(w: *mut lp_pack_writer) -> c_int;
    pub fn lp_pack_open(path: *const c_char, direct: c_int, out: *mut *mut lp_pack) -> c_int;
    pub fn lp_pack_close(p: *mut lp_pack);
    pub fn lp_pack_info(p: *const lp_pack, layers: *mut u32, experts: *mut u32, max_blob_bytes: *mut u64) -> c_int;
    pub fn lp_pack_entry(p: *const lp_pack, layer: u32, expert: u32, offset: *mut u64, nbytes: *mut u64) -> c_int;
    pub fn lp_pack_read_blob(p: *mut lp_pack, layer: u32, expert: u32, buf: *mut c_void, buf_len: u64) -> i64;

    // ---- blob format ----
    pub fn lp_q4_bytes(rows: c_int, cols: c_int, group: c_int) -> u64;
    pub fn lp_blob_bytes(hidden: c_int, inter: c_int, group: c_int) -> u64;
    pub fn lp_blob_offsets(hidden: c_int, inter: c_int, group: c_int, gate: *mut u64, up: *mut u64, down: *mut u64);
}

/// `driver.rs:20-27`'s convention: a non-zero return is an error carrying
/// this thread's `lp_last_error()` text.
pub fn check(rc: c_int, name: &str) -> anyhow::Result<()> {
    if rc == 0 {
        return Ok(());
    }
    let msg = unsafe { std::ffi::CStr::from_ptr(lp_last_error()) }.to_string_lossy().into_owned();
    anyhow::bail!("{name} failed: llmpager_hip error {rc} ({msg})")
}
