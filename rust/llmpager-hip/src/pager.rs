//! Expert pager over the C ABI: the surface of `pager::Pager`
//! (`crates/llmpager-cuda/src/pager.rs`).  The workers, staging rings, RAM
//! tier, slot cache and the VRAM reserve (`lp_pager_config::reserve_bytes`)
//! live in the library (`lp_pager_open`); this module keeps the reference's
//! types and method names.
use std::ffi::CString;
use std::os::unix::ffi::OsStrExt;
use std::path::Path;
use std::sync::Arc;

use anyhow::Result;

use crate::driver::{CUdeviceptr, CUstream, Cuda};
use crate::ffi::{self, check};

/// `pager.rs:33-63`, same fields and defaults.
#[derive(Clone, Debug)]
pub struct PagerConfig {
    pub slots_per_layer: u32,
    pub io_threads: usize,
    /// Per-layer pools halve their frequency counters every this many
    /// insertions.
    pub decay_interval: u32,
    /// Pack reads with O_DIRECT (bypassing the page cache).
    pub direct: bool,
    /// Host-RAM expert tier in bytes, 0 = none.
    pub ram_bytes: u64,
    /// VRAM to leave free on the card; `slots_per_layer` is clamped to fit.
    pub reserve_bytes: u64,
}

impl Default for PagerConfig {
    fn default() -> Self {
        Self { slots_per_layer: 32, io_threads: 4, decay_interval: 256, direct: true, ram_bytes: 0, reserve_bytes: 0 }
    }
}

/// `pager.rs:169-178`: a pinned expert, resident or in flight.  Drop does
/// not release it; hand it to [`Pager::release`].
#[derive(Debug)]
pub struct ExpertHandle {
    pub layer: u16,
    pub expert: u16,
    pub slot: u32,
    /// Device address of the expert's blob.
    pub dev: CUdeviceptr,
    /// Valid bytes at `dev`.
    pub len: usize,
}

/// `pager.rs:622-652`.
#[derive(Debug, Clone)]
pub struct Metrics {
    pub hits: u64,
    pub misses: u64,
    pub bytes_fetched: u64,
    pub fetches: u64,
    /// Fetches served from the host-RAM tier (a subset of `fetches`).
    pub ram_hits: u64,
    /// Fetch wall-time histogram: <1, <2, <5, <10, <20, <50, >=50 ms.
    pub latency_ms_buckets: [u64; 7],
}

/// Upper edges (ms) of the fetch-time buckets; the last bucket is open.
const LATENCY_EDGES_MS: [u32; 6] = [1, 2, 5, 10, 20, 50];

impl Metrics {
    /// Hits over all lookups; 0 before the first lookup.
    pub fn hit_rate(&self) -> f64 {
        match self.hits + self.misses {
            0 => 0.0,
            lookups => self.hits as f64 / lookups as f64,
        }
    }

    /// The fetch-time buckets as `<edge>ms:count` pairs, the open last one
    /// as `>=50ms:count`.
    pub fn histogram(&self) -> String {
        let mut out = String::new();
        for (i, count) in self.latency_ms_buckets.iter().enumerate() {
            let label = match LATENCY_EDGES_MS.get(i) {
                Some(edge) => format!("<{edge}ms"),
                None => format!(">={}ms", LATENCY_EDGES_MS[LATENCY_EDGES_MS.len() - 1]),
            };
            if i > 0 {
                out.push(' ');
            }
            out.push_str(&label);
            out.push(':');
            out.push_str(&count.to_string());
        }
        out
    }
}

pub struct Pager {
    // keeps the context alive for as long as the pager's workers use it
    _cuda: Arc<Cuda>,
    p: *mut ffi::lp_pager,
    layers: u32,
    experts_per_layer: u32,
}

unsafe impl Send for Pager {}
unsafe impl Sync for Pager {}

impl Pager {
    /// `pager.rs:260-388`: open `pack`, allocate the arena (its slot count
    /// lowered by the library until `reserve_bytes` stay free: read it back
    /// with [`Pager::slots_per_layer`]) and start `io_threads` workers.
    /// `LLMPAGER_GLOBAL_POOL=1` selects one pool shared by every layer.
    pub fn new(cuda: Arc<Cuda>, pack: &Path, cfg: PagerConfig) -> Result<Self> {
        let path = CString::new(pack.as_os_str().as_bytes())?;
        // the pack's shape (for expert_stats); the library reads it again
        let (mut layers, mut experts, mut max_blob) = (0u32, 0u32, 0u64);
        {
            let mut pk = std::ptr::null_mut();
            check(unsafe { ffi::lp_pack_open(path.as_ptr(), 0, &mut pk) }, "lp_pack_open")?;
            let rc = unsafe { ffi::lp_pack_info(pk, &mut layers, &mut experts, &mut max_blob) };
            unsafe { ffi::lp_pack_close(pk) };
            check(rc, "lp_pack_info")?;
        }
        let global_pool = std::env::var("LLMPAGER_GLOBAL_POOL").ok().as_deref() == Some("1");
        let c = ffi::lp_pager_config {
            layers,
            experts_per_layer: experts,
            slots_per_layer: cfg.slots_per_layer,
            decay_interval: cfg.decay_interval,
            blob_bytes: 0,
            span: 0,
            host_blobs: std::ptr::null(),
            host_stride: 0,
            copy_streams: 0,
            global_pool: global_pool as i32,
            pool_decay_tokens: 0,
            source: ffi::LP_PAGER_SRC_PACK,
            direct: cfg.direct as i32,
            io_threads: cfg.io_threads as u32,
            ring_slots: 0,
            stage_threads: 0,
            ram_bytes: cfg.ram_bytes,
            reserve_bytes: cfg.reserve_bytes,
        };
        let mut p = std::ptr::null_mut();
        check(unsafe { ffi::lp_pager_open(cuda.ctx, path.as_ptr(), &c, &mut p) }, "lp_pager_open")?;
        Ok(Self { _cuda: cuda, p, layers, experts_per_layer: experts })
    }

    /// `pager.rs:402-460`: pin every expert, schedule the misses, return at
    /// once; blocks only while the layer's pool is entirely pinned.
    pub fn request(&self, layer: u16, experts: &[u16]) -> Result<Vec<ExpertHandle>> {
        let mut raw = vec![ffi::lp_expert_handle::default(); experts.len()];
        let rc = unsafe {
            ffi::lp_pager_request_handles(self.p, layer, experts.as_ptr(), experts.len() as i32, raw.as_mut_ptr())
        };
        check(rc, "Pager::request")?;
        Ok(raw
            .into_iter()
            .map(|h| ExpertHandle { layer: h.layer, expert: h.expert, slot: h.slot, dev: h.dev, len: h.len as usize })
            .collect())
    }

    /// `pager.rs:464-486`: best effort, never blocks.
    pub fn prefetch(&self, layer: u16, experts: &[u16]) {
        unsafe { ffi::lp_pager_prefetch(self.p, layer, experts.as_ptr(), experts.len() as i32) };
    }

    /// `pager.rs:487-495`: block the host until the expert is in VRAM.
    pub fn wait(&self, h: &ExpertHandle) -> Result<()> {
        check(unsafe { ffi::lp_pager_wait(self.p, h.slot) }, "Pager::wait")
    }

    /// `pager.rs:497-503`: make `stream` wait for the expert's copy.
    pub fn wait_stream(&self, h: &ExpertHandle, stream: CUstream) -> Result<()> {
        let raw = ffi::lp_expert_handle { layer: h.layer, expert: h.expert, slot: h.slot, dev: h.dev, len: h.len as u64 };
        check(unsafe { ffi::lp_pager_wait_stream(self.p, &raw, stream) }, "Pager::wait_stream")
    }

    /// Refresh `layer`'s device slot table on `stream`, in stream order,
    /// for the fused layer kernels that read it.
    pub fn refresh_table(&self, layer: u16, stream: CUstream) -> Result<()> {
        check(unsafe { ffi::lp_pager_refresh_table(self.p, layer, stream) }, "Pager::refresh_table")
    }

    /// `pager.rs:505-510`.
    pub fn release(&self, h: ExpertHandle) {
        unsafe { ffi::lp_pager_release(self.p, &h.slot, 1) };
    }

    /// Unpin once `stream` has passed this point (the deferred release of
    /// `decode.rs:621-649`).
    pub fn release_after(&self, hs: Vec<ExpertHandle>, stream: CUstream) -> Result<()> {
        let slots: Vec<u32> = hs.iter().map(|h| h.slot).collect();
        check(unsafe { ffi::lp_pager_release_after(self.p, slots.as_ptr(), slots.len() as i32, stream) }, "release_after")
    }

    pub fn slots_per_layer(&self) -> u32 {
        unsafe { ffi::lp_pager_slots_per_layer(self.p) }
    }

    /// `pager.rs:521-530`: end of a forward pass (global-pool decay).
    pub fn tick(&self) {
        unsafe { ffi::lp_pager_tick(self.p) };
    }

    /// `pager.rs:532-535`: fills per (layer, expert), row-major.
    pub fn expert_stats(&self) -> Vec<u64> {
        let mut v = vec![0u64; self.layers as usize * self.experts_per_layer as usize];
        unsafe { ffi::lp_pager_expert_stats(self.p, v.as_mut_ptr(), v.len() as u64) };
        v
    }

    /// `pager.rs:540-567`: read the most-fetched experts of `counts` into
    /// the RAM tier; returns how many (0 without one).
    pub fn prewarm(&self, counts: &[u64]) -> Result<usize> {
        let rc = unsafe { ffi::lp_pager_prewarm(self.p, counts.as_ptr(), counts.len() as u64) };
        if rc < 0 {
            check(rc, "Pager::prewarm")?;
        }
        Ok(rc as usize)
    }

    /// `pager.rs:568-589`.
    pub fn metrics(&self) -> Metrics {
        let mut m = ffi::lp_pager_metrics::default();
        unsafe { ffi::lp_pager_get_metrics(self.p, &mut m) };
        Metrics {
            hits: m.hits,
            misses: m.misses,
            bytes_fetched: m.bytes_fetched,
            fetches: m.fetches,
            ram_hits: m.ram_hits,
            latency_ms_buckets: m.latency_ms_buckets,
        }
    }

    /// The arena base, slot span and `layer`'s device slot table: the
    /// fields a [`crate::MoeLayerDesc`] takes from the pager.
    pub fn arena(&self) -> (CUdeviceptr, u64) {
        unsafe { (ffi::lp_pager_arena(self.p), ffi::lp_pager_span(self.p)) }
    }

    pub fn slot_table(&self, layer: u32) -> CUdeviceptr {
        unsafe { ffi::lp_pager_slot_table(self.p, layer) }
    }
}

impl Drop for Pager {
    /// `pager.rs:606-620`: stop the workers, wait for copies in flight.
    fn drop(&mut self) {
        unsafe { ffi::lp_pager_free(self.p) };
    }
}
