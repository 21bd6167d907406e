//! Hot-path launchers: the surface of `kernels::Kernels`
//! (`crates/llmpager-cuda/src/kernels.rs`), one method per reference
//! method with the same argument order and meaning, each a call into the
//! library's gfx950 launcher (`include/llmpager_hip.h` cites the reference
//! line each replaces).  The fused MoE layer entries (`moe_*`, `stack_*`)
//! have no reference method: they replace the per-expert sequence the
//! reference's decode loop issues (`decode.rs:734-790`).
use anyhow::{bail, Result};

use crate::driver::{CUdeviceptr, CUstream, Cuda};
use crate::ffi::{self, check, lp_moe_layer_desc, lp_moe_ws_layout};

/// The code objects are loaded by [`Cuda::init`]; `Kernels` keeps the
/// reference's shape (`load`, then `&self` methods taking `&Cuda`).
pub struct Kernels {
    _priv: (),
}

/// A captured HIP graph (`lp_moe_stack_capture`, `lp_graph_capture_end`).
pub struct Graph {
    g: *mut ffi::lp_graph,
}

impl Drop for Graph {
    fn drop(&mut self) {
        unsafe { ffi::lp_graph_destroy(self.g) };
    }
}

unsafe impl Send for Graph {}

impl Kernels {
    /// `kernels.rs:44-68`.
    pub fn load(_cuda: &Cuda) -> Result<Self> {
        Ok(Self { _priv: () })
    }

    #[allow(clippy::too_many_arguments)]
    pub fn q4g64_gemv(
        &self, cuda: &Cuda, blob: CUdeviceptr, x: CUdeviceptr, y: CUdeviceptr, rows: i32, cols: i32, group: i32,
        stream: CUstream,
    ) -> Result<()> {
        check(unsafe { ffi::lp_q4_gemv(cuda.ctx, blob, x, y, rows, cols, group, stream) }, "q4g64_gemv")
    }

    #[allow(clippy::too_many_arguments)]
    pub fn q4g64_gemv_batch(
        &self, cuda: &Cuda, blobs: CUdeviceptr, region_off: u64, x: CUdeviceptr, x_stride: i32, y: CUdeviceptr,
        rows: i32, cols: i32, group: i32, experts: i32, stream: CUstream,
    ) -> Result<()> {
        let rc = unsafe {
            ffi::lp_q4_gemv_batch(cuda.ctx, blobs, region_off, x, x_stride, y, rows, cols, group, experts, stream)
        };
        check(rc, "q4g64_gemv_batch")
    }

    #[allow(clippy::too_many_arguments)]
    pub fn moe_reduce(
        &self, cuda: &Cuda, eouts: CUdeviceptr, wts: CUdeviceptr, out: CUdeviceptr, experts: i32, n: i32,
        stream: CUstream,
    ) -> Result<()> {
        check(unsafe { ffi::lp_moe_reduce(cuda.ctx, eouts, wts, out, experts, n, stream) }, "moe_reduce")
    }

    #[allow(clippy::too_many_arguments)]
    pub fn rmsnorm(
        &self, cuda: &Cuda, x: CUdeviceptr, w: CUdeviceptr, y: CUdeviceptr, rows: i32, n: i32, eps: f32,
        stream: CUstream,
    ) -> Result<()> {
        check(unsafe { ffi::lp_rmsnorm(cuda.ctx, x, w, y, rows, n, eps, stream) }, "rmsnorm")
    }

    pub fn scale_add(&self, cuda: &Cuda, a: CUdeviceptr, b: CUdeviceptr, s: f32, n: i32, stream: CUstream) -> Result<()> {
        check(unsafe { ffi::lp_scale_add(cuda.ctx, a, b, s, n, stream) }, "scale_add")
    }

    #[allow(clippy::too_many_arguments)]
    pub fn kv_append(
        &self, cuda: &Cuda, k: CUdeviceptr, v: CUdeviceptr, kcache: CUdeviceptr, vcache: CUdeviceptr, kv_heads: i32,
        head_dim: i32, pos: i32, max_seq: i32, f16: bool, stream: CUstream,
    ) -> Result<()> {
        let rc = unsafe {
            ffi::lp_kv_append(cuda.ctx, k, v, kcache, vcache, kv_heads, head_dim, pos, max_seq, f16 as i32, stream)
        };
        check(rc, "kv_append")
    }

    #[allow(clippy::too_many_arguments)]
    pub fn bf16_gemv(
        &self, cuda: &Cuda, w: CUdeviceptr, x: CUdeviceptr, y: CUdeviceptr, rows: i32, cols: i32, stream: CUstream,
    ) -> Result<()> {
        check(unsafe { ffi::lp_bf16_gemv(cuda.ctx, w, x, y, rows, cols, stream) }, "bf16_gemv")
    }

    #[allow(clippy::too_many_arguments)]
    pub fn silu_mul(
        &self, cuda: &Cuda, gate: CUdeviceptr, up: CUdeviceptr, out: CUdeviceptr, n: i32, stream: CUstream,
    ) -> Result<()> {
        check(unsafe { ffi::lp_silu_mul(cuda.ctx, gate, up, out, n, stream) }, "silu_mul")
    }

    /// `a += b` (`kernels.rs:239-251`).
    pub fn add(&self, cuda: &Cuda, a: CUdeviceptr, b: CUdeviceptr, n: i32, stream: CUstream) -> Result<()> {
        check(unsafe { ffi::lp_add(cuda.ctx, a, b, n, stream) }, "add")
    }

    #[allow(clippy::too_many_arguments)]
    pub fn rope(
        &self, cuda: &Cuda, x: CUdeviceptr, heads: i32, head_dim: i32, pos: i32, base: f32, stream: CUstream,
    ) -> Result<()> {
        check(unsafe { ffi::lp_rope(cuda.ctx, x, heads, head_dim, pos, base, stream) }, "rope")
    }

    #[allow(clippy::too_many_arguments)]
    pub fn attn_decode(
        &self, cuda: &Cuda, q: CUdeviceptr, kcache: CUdeviceptr, vcache: CUdeviceptr, out: CUdeviceptr,
        scratch: CUdeviceptr, heads: i32, kv_heads: i32, head_dim: i32, seq_len: i32, max_seq: i32, scale: f32,
        f16: bool, stream: CUstream,
    ) -> Result<()> {
        let rc = unsafe {
            ffi::lp_attn_decode(
                cuda.ctx, q, kcache, vcache, out, scratch, heads, kv_heads, head_dim, seq_len, max_seq, scale,
                f16 as i32, stream,
            )
        };
        check(rc, "attn_decode")
    }

    #[allow(clippy::too_many_arguments)]
    pub fn bf16_row(
        &self, cuda: &Cuda, table: CUdeviceptr, row: i32, n: i32, out: CUdeviceptr, stream: CUstream,
    ) -> Result<()> {
        check(unsafe { ffi::lp_bf16_row(cuda.ctx, table, row, n, out, stream) }, "bf16_row")
    }

    /// `y_i = W_i . rmsnorm(x, ln)` for one to three bf16 matrices `(w, rows, y)`
    /// sharing `x` (`ln` 0: no norm).  No `kernels.rs` counterpart: the
    /// rmsnorm and bf16_gemv launches of `decode.rs:282-285, 359-360` in one.
    #[allow(clippy::too_many_arguments)]
    pub fn rmsnorm_gemv(
        &self, cuda: &Cuda, x: CUdeviceptr, ln: CUdeviceptr, eps: f32, cols: i32,
        mats: &[(CUdeviceptr, i32, CUdeviceptr)], stream: CUstream,
    ) -> Result<()> {
        if mats.is_empty() || mats.len() > 3 {
            bail!("rmsnorm_gemv takes one to three matrices");
        }
        let m = |i: usize| mats.get(i).copied().unwrap_or((0, 0, 0));
        let (a, b, c) = (m(0), m(1), m(2));
        let rc = unsafe {
            ffi::lp_rmsnorm_gemv(cuda.ctx, x, ln, eps, cols, a.0, a.1, a.2, b.0, b.1, b.2, c.0, c.1, c.2, stream)
        };
        check(rc, "rmsnorm_gemv")
    }

    /// `h += W . x`, then `hn = rmsnorm(h, ln)` (`decode.rs:296-301` in one launch).
    #[allow(clippy::too_many_arguments)]
    pub fn gemv_add_rmsnorm(
        &self, cuda: &Cuda, w: CUdeviceptr, x: CUdeviceptr, rows: i32, cols: i32, h: CUdeviceptr,
        ln: CUdeviceptr, eps: f32, hn: CUdeviceptr, stream: CUstream,
    ) -> Result<()> {
        let rc = unsafe { ffi::lp_gemv_add_rmsnorm(cuda.ctx, w, x, rows, cols, h, ln, eps, hn, stream) };
        check(rc, "gemv_add_rmsnorm")
    }

    /// Per-head q / k rmsnorm, rope, the fp16 KV append at `pos` and GQA decode
    /// attention over `pos + 1` positions (`decode.rs:283-294` in one launch).
    #[allow(clippy::too_many_arguments)]
    pub fn attn_fused(
        &self, cuda: &Cuda, q: CUdeviceptr, k: CUdeviceptr, v: CUdeviceptr, q_norm: CUdeviceptr,
        k_norm: CUdeviceptr, eps: f32, rope_base: f32, kcache: CUdeviceptr, vcache: CUdeviceptr, out: CUdeviceptr,
        scratch: CUdeviceptr, heads: i32, kv_heads: i32, head_dim: i32, pos: i32, max_seq: i32, scale: f32,
        stream: CUstream,
    ) -> Result<()> {
        let rc = unsafe {
            ffi::lp_attn_fused(
                cuda.ctx, q, k, v, q_norm, k_norm, eps, rope_base, kcache, vcache, out, scratch, heads, kv_heads,
                head_dim, pos, max_seq, scale, stream,
            )
        };
        check(rc, "attn_fused")
    }

    /// `attn_fused` into `att`, then `h += W_o . att` and `hn = rmsnorm(h, post_ln)`
    /// in one launch (`decode.rs:283-301`).
    #[allow(clippy::too_many_arguments)]
    pub fn attn_block(
        &self, cuda: &Cuda, q: CUdeviceptr, k: CUdeviceptr, v: CUdeviceptr, q_norm: CUdeviceptr,
        k_norm: CUdeviceptr, eps: f32, rope_base: f32, kcache: CUdeviceptr, vcache: CUdeviceptr, att: CUdeviceptr,
        scratch: CUdeviceptr, heads: i32, kv_heads: i32, head_dim: i32, pos: i32, max_seq: i32, scale: f32,
        wo: CUdeviceptr, h: CUdeviceptr, post_ln: CUdeviceptr, hn: CUdeviceptr, hidden: i32, stream: CUstream,
    ) -> Result<()> {
        let rc = unsafe {
            ffi::lp_attn_block(
                cuda.ctx, q, k, v, q_norm, k_norm, eps, rope_base, kcache, vcache, att, scratch, heads, kv_heads,
                head_dim, pos, max_seq, scale, wo, h, post_ln, hn, hidden, stream,
            )
        };
        check(rc, "attn_block")
    }

    #[allow(clippy::too_many_arguments)]
    pub fn mla_rope(
        &self, cuda: &Cuda, x: CUdeviceptr, n_vecs: i32, stride: i32, offset: i32, half: i32, pos: i32,
        inv_freq: CUdeviceptr, mscale: f32, stream: CUstream,
    ) -> Result<()> {
        let rc = unsafe { ffi::lp_mla_rope(cuda.ctx, x, n_vecs, stride, offset, half, pos, inv_freq, mscale, stream) };
        check(rc, "mla_rope")
    }

    #[allow(clippy::too_many_arguments)]
    pub fn mla_attn_decode(
        &self, cuda: &Cuda, q: CUdeviceptr, cache: CUdeviceptr, ctx: CUdeviceptr, scratch: CUdeviceptr, heads: i32,
        qk_dim: i32, c_dim: i32, seq_len: i32, max_seq: i32, scale: f32, stream: CUstream,
    ) -> Result<()> {
        let rc = unsafe {
            ffi::lp_mla_attn_decode(cuda.ctx, q, cache, ctx, scratch, heads, qk_dim, c_dim, seq_len, max_seq, scale, stream)
        };
        check(rc, "mla_attn_decode")
    }

    #[allow(clippy::too_many_arguments)]
    pub fn bf16_gemv_batch(
        &self, cuda: &Cuda, w: CUdeviceptr, w_stride: u64, x: CUdeviceptr, x_stride: i32, y: CUdeviceptr,
        y_stride: i32, rows: i32, cols: i32, batch: i32, stream: CUstream,
    ) -> Result<()> {
        let rc = unsafe {
            ffi::lp_bf16_gemv_batch(cuda.ctx, w, w_stride, x, x_stride, y, y_stride, rows, cols, batch, stream)
        };
        check(rc, "bf16_gemv_batch")
    }

    #[allow(clippy::too_many_arguments)]
    pub fn strided_copy(
        &self, cuda: &Cuda, src: CUdeviceptr, src_stride: i32, src_off: i32, dst: CUdeviceptr, dst_stride: i32,
        dst_off: i32, n_vecs: i32, n: i32, stream: CUstream,
    ) -> Result<()> {
        let rc = unsafe {
            ffi::lp_strided_copy(cuda.ctx, src, src_stride, src_off, dst, dst_stride, dst_off, n_vecs, n, stream)
        };
        check(rc, "strided_copy")
    }

    // ---- beyond the reference's launchers ----

    /// Workspace bytes for [`Self::mla_attn_decode_batch`].
    pub fn mla_batch_ws_bytes(&self, cuda: &Cuda, batch: i32, c_dim: i32, max_seq: i32) -> u64 {
        unsafe { ffi::lp_mla_batch_ws_bytes(cuda.ctx, batch, c_dim, max_seq) }
    }

    /// MLA absorbed decode for `batch` sequences over bf16 latent caches
    /// (`seq_lens`: device i32 [batch]) on the matrix cores.
    #[allow(clippy::too_many_arguments)]
    pub fn mla_attn_decode_batch(
        &self, cuda: &Cuda, q: CUdeviceptr, cache: CUdeviceptr, cache_stride: u64, seq_lens: CUdeviceptr,
        ctx: CUdeviceptr, workspace: CUdeviceptr, batch: i32, heads: i32, qk_dim: i32, c_dim: i32, max_seq: i32,
        scale: f32, stream: CUstream,
    ) -> Result<()> {
        let rc = unsafe {
            ffi::lp_mla_attn_decode_batch(
                cuda.ctx, q, cache, cache_stride, seq_lens, ctx, workspace, batch, heads, qk_dim, c_dim, max_seq,
                scale, stream,
            )
        };
        check(rc, "mla_attn_decode_batch")
    }

    /// Workspace layout (and `total` bytes) of one MoE layer over `t` tokens.
    pub fn moe_ws_layout(&self, d: &lp_moe_layer_desc, t: i32) -> Result<lp_moe_ws_layout> {
        let mut out = lp_moe_ws_layout::default();
        check(unsafe { ffi::lp_moe_ws_layout_get(d, t, &mut out) }, "moe_ws_layout")?;
        Ok(out)
    }

    /// The workspace check every MoE entry point makes before launching
    /// (`ws_bytes` at least the largest layer's layout total), on its own.
    pub fn moe_workspace_check(&self, layers: &[lp_moe_layer_desc], t: i32, ws: CUdeviceptr, ws_bytes: u64) -> Result<()> {
        let rc = unsafe { ffi::lp_moe_workspace_check(layers.as_ptr(), layers.len() as i32, t, ws, ws_bytes) };
        check(rc, "moe_workspace_check")
    }

    /// Routing alone: router GEMV, top-k, dispatch groups into `ws`
    /// (`ws_bytes` long).
    #[allow(clippy::too_many_arguments)]
    pub fn moe_route(
        &self, cuda: &Cuda, d: &lp_moe_layer_desc, x: CUdeviceptr, t: i32, ws: CUdeviceptr, ws_bytes: u64,
        stream: CUstream,
    ) -> Result<()> {
        check(unsafe { ffi::lp_moe_route(cuda.ctx, d, x, t, ws, ws_bytes, stream) }, "moe_route")
    }

    /// Routing from caller-supplied router logits (f32 [t, experts]).
    #[allow(clippy::too_many_arguments)]
    pub fn moe_route_logits(
        &self, cuda: &Cuda, d: &lp_moe_layer_desc, logits: CUdeviceptr, t: i32, ws: CUdeviceptr, ws_bytes: u64,
        stream: CUstream,
    ) -> Result<()> {
        check(unsafe { ffi::lp_moe_route_logits(cuda.ctx, d, logits, t, ws, ws_bytes, stream) }, "moe_route_logits")
    }

    /// Paged flow: after routing and the pager's requests for the picks,
    /// re-resolve the expert entries through the now-current slot table.
    pub fn moe_resolve(
        &self, cuda: &Cuda, d: &lp_moe_layer_desc, t: i32, ws: CUdeviceptr, ws_bytes: u64, stream: CUstream,
    ) -> Result<()> {
        check(unsafe { ffi::lp_moe_resolve(cuda.ctx, d, t, ws, ws_bytes, stream) }, "moe_resolve")
    }

    /// The expert half of a routed layer: `h += sum_k w * expert_k(x)`.
    #[allow(clippy::too_many_arguments)]
    pub fn moe_experts(
        &self, cuda: &Cuda, d: &lp_moe_layer_desc, x: CUdeviceptr, h: CUdeviceptr, t: i32, ws: CUdeviceptr,
        ws_bytes: u64, stream: CUstream,
    ) -> Result<()> {
        check(unsafe { ffi::lp_moe_experts(cuda.ctx, d, x, h, t, ws, ws_bytes, stream) }, "moe_experts")
    }

    /// One wave of a paged union (`decode.rs:483-531`): the routed experts
    /// `uniq[u_first .. u_first + u_count)` of the dispatch's unique list,
    /// each token's picks among them summed in pick order and added into `h`
    /// once; `with_shared` adds the shared MLP after them (the last wave).
    #[allow(clippy::too_many_arguments)]
    pub fn moe_experts_wave(
        &self, cuda: &Cuda, d: &lp_moe_layer_desc, x: CUdeviceptr, h: CUdeviceptr, t: i32, ws: CUdeviceptr,
        ws_bytes: u64, u_first: i32, u_count: i32, with_shared: bool, stream: CUstream,
    ) -> Result<()> {
        let rc = unsafe {
            ffi::lp_moe_experts_wave(cuda.ctx, d, x, h, t, ws, ws_bytes, u_first, u_count, with_shared as i32, stream)
        };
        check(rc, "moe_experts_wave")
    }

    /// One whole MoE layer: route, gate/up, SiLU, down, weighted combine
    /// into `h` (`x` = the normalised input, f32 [t, hidden]).
    #[allow(clippy::too_many_arguments)]
    pub fn moe_forward(
        &self, cuda: &Cuda, d: &lp_moe_layer_desc, x: CUdeviceptr, h: CUdeviceptr, t: i32, ws: CUdeviceptr,
        ws_bytes: u64, stream: CUstream,
    ) -> Result<()> {
        check(unsafe { ffi::lp_moe_forward(cuda.ctx, d, x, h, t, ws, ws_bytes, stream) }, "moe_forward")
    }

    /// [`Self::moe_forward`] with its workspace in the library's own
    /// device scratch: no allocation, for callers that cannot allocate.
    pub fn moe_forward_noalloc(
        &self, cuda: &Cuda, d: &lp_moe_layer_desc, x: CUdeviceptr, h: CUdeviceptr, t: i32, stream: CUstream,
    ) -> Result<()> {
        check(unsafe { ffi::lp_moe_forward_noalloc(cuda.ctx, d, x, h, t, stream) }, "moe_forward_noalloc")
    }

    /// A stack of MoE layers over the residual `h` (f32 [t, hidden]).
    #[allow(clippy::too_many_arguments)]
    pub fn stack_forward(
        &self, cuda: &Cuda, layers: &[lp_moe_layer_desc], h: CUdeviceptr, t: i32, ws: CUdeviceptr, ws_bytes: u64,
        stream: CUstream,
    ) -> Result<()> {
        let rc = unsafe {
            ffi::lp_moe_stack_forward(cuda.ctx, layers.as_ptr(), layers.len() as i32, h, t, ws, ws_bytes, stream)
        };
        check(rc, "stack_forward")
    }

    /// [`Self::stack_forward`] captured once into a HIP graph.
    #[allow(clippy::too_many_arguments)]
    pub fn stack_capture(
        &self, cuda: &Cuda, layers: &[lp_moe_layer_desc], h: CUdeviceptr, t: i32, ws: CUdeviceptr, ws_bytes: u64,
        stream: CUstream,
    ) -> Result<Graph> {
        let mut g = std::ptr::null_mut();
        let rc = unsafe {
            ffi::lp_moe_stack_capture(
                cuda.ctx, layers.as_ptr(), layers.len() as i32, h, t, ws, ws_bytes, stream, &mut g,
            )
        };
        check(rc, "stack_capture")?;
        Ok(Graph { g })
    }

    /// Start recording every launch made on `stream` (a whole decode step:
    /// the attention block's kernels and the MoE layers) into one graph.
    pub fn capture_begin(&self, cuda: &Cuda, stream: CUstream) -> Result<()> {
        check(unsafe { ffi::lp_graph_capture_begin(cuda.ctx, stream) }, "capture_begin")
    }

    /// End the recording started by [`Self::capture_begin`].
    pub fn capture_end(&self, cuda: &Cuda, stream: CUstream) -> Result<Graph> {
        let mut g = std::ptr::null_mut();
        check(unsafe { ffi::lp_graph_capture_end(cuda.ctx, stream, &mut g) }, "capture_end")?;
        Ok(Graph { g })
    }

    pub fn graph_launch(&self, cuda: &Cuda, g: &Graph, stream: CUstream) -> Result<()> {
        check(unsafe { ffi::lp_graph_launch(cuda.ctx, g.g, stream) }, "graph_launch")
    }

    /// Synchronise `stream` and read the layer's (unique experts, error
    /// flags); a non-zero flag word is an error.
    pub fn moe_status(
        &self, cuda: &Cuda, ws: CUdeviceptr, ws_bytes: u64, d: &lp_moe_layer_desc, t: i32, stream: CUstream,
    ) -> Result<i32> {
        let (mut uniq, mut flags) = (0i32, 0i32);
        let rc = unsafe { ffi::lp_moe_status_sync(cuda.ctx, ws, ws_bytes, d, t, stream, &mut uniq, &mut flags) };
        check(rc, "moe_status")?;
        anyhow::ensure!(flags == 0, "MoE layer reported error flags {flags:#x}");
        Ok(uniq)
    }
}
