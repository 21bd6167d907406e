//! MI355X (gfx950) side of llmpager, over the `llmpager_hip` C ABI
//! (`include/llmpager_hip.h`, built by `llmpager_amd/build.py`).
//!
//! The module layout and public surface follow `crates/llmpager-cuda`
//! (`lib.rs:1-15`) so that a caller switches crates without other changes:
//! [`driver`] is the device runtime (`driver::Cuda`, `Pinned`, the
//! `CUdeviceptr`/`CUstream`/`CUevent` aliases), [`kernels`] the hot-path
//! launchers (`kernels::Kernels`, every method of the reference's plus the
//! fused MoE layer entries), [`pager`] the expert pager (`pager::Pager`,
//! `PagerConfig`, `ExpertHandle`, `Metrics`).  All device work happens in
//! the shared library; this crate only marshals arguments and turns return
//! codes into `anyhow` errors.

pub mod driver;
mod ffi;
#[cfg(feature = "kernels")]
pub mod kernels;
pub mod pager;

pub use ffi::{lp_moe_layer_desc as MoeLayerDesc, lp_moe_ws_layout as MoeWsLayout};
