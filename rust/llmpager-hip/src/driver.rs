//! Device runtime over the C ABI: the surface of `driver::Cuda`
//! (`crates/llmpager-cuda/src/driver.rs:29-304`).  The reference loads
//! `libcuda.so.1` and JIT-loads PTX; here `lp_init` makes the device current
//! and loads the gfx950 code objects, so `module_from_ptx`, `function` and
//! `launch` have no counterpart — every kernel has its own launcher in
//! [`crate::kernels`].
use std::ffi::CString;
use std::os::raw::c_void;
use std::ptr;

use anyhow::Result;

use crate::ffi::{self, check};

/// Device addresses are plain integers, as in `driver.rs:10`.
pub type CUdeviceptr = u64;
/// A `hipStream_t`; null is the null stream (`driver.rs:11`).
pub type CUstream = *mut c_void;
/// A `hipEvent_t` (`driver.rs:12`).
pub type CUevent = *mut c_void;

pub struct Cuda {
    pub(crate) ctx: *mut ffi::lp_ctx,
}

impl Cuda {
    /// `driver.rs:66-112`: device `LLMPAGER_HIP_DEVICE` (default 0); the
    /// code objects come from `LLMPAGER_HIP_HSACO` or, unset, the directory
    /// the shared library was loaded from.
    pub fn init() -> Result<Self> {
        let device = std::env::var("LLMPAGER_HIP_DEVICE").ok().and_then(|s| s.parse().ok()).unwrap_or(0);
        let dir = std::env::var("LLMPAGER_HIP_HSACO").ok().map(CString::new).transpose()?;
        Self::init_on(device, dir.as_deref())
    }

    pub fn init_on(device: i32, hsaco_dir: Option<&std::ffi::CStr>) -> Result<Self> {
        let mut ctx = ptr::null_mut();
        let dir = hsaco_dir.map_or(ptr::null(), |d| d.as_ptr());
        check(unsafe { ffi::lp_init(device, dir, &mut ctx) }, "lp_init")?;
        Ok(Self { ctx })
    }

    /// `driver.rs:117-123`: (free, total) bytes.
    pub fn mem_info(&self) -> Result<(u64, u64)> {
        let (mut free, mut total) = (0u64, 0u64);
        check(unsafe { ffi::lp_mem_info(self.ctx, &mut free, &mut total) }, "lp_mem_info")?;
        Ok((free, total))
    }

    /// `driver.rs:125-129`: make this context's device current on the
    /// calling thread (worker threads call it first).
    pub fn bind_thread(&self) -> Result<()> {
        check(unsafe { ffi::lp_bind_thread(self.ctx) }, "lp_bind_thread")
    }

    pub fn alloc_device(&self, len: usize) -> Result<CUdeviceptr> {
        let mut p = 0u64;
        check(unsafe { ffi::lp_alloc_device(self.ctx, len, &mut p) }, "lp_alloc_device")?;
        Ok(p)
    }

    /// `driver.rs:137-141`: errors are dropped, as the reference drops them.
    pub fn free_device(&self, p: CUdeviceptr) {
        unsafe { ffi::lp_free_device(self.ctx, p) };
    }

    /// `driver.rs:143-147`: page-locked host memory (`hipHostMalloc`).
    pub fn alloc_pinned(&self, len: usize) -> Result<Pinned> {
        let mut p = ptr::null_mut();
        check(unsafe { ffi::lp_alloc_pinned(self.ctx, len, &mut p) }, "lp_alloc_pinned")?;
        Ok(Pinned { ptr: p as *mut u8, len })
    }

    pub fn free_pinned(&self, b: &Pinned) {
        unsafe { ffi::lp_free_pinned(self.ctx, b.ptr as *mut c_void) };
    }

    /// `driver.rs:153-157`: a non-blocking stream at the default priority.
    pub fn stream(&self) -> Result<CUstream> {
        let mut s = ptr::null_mut();
        check(unsafe { ffi::lp_stream_create(self.ctx, &mut s) }, "lp_stream_create")?;
        Ok(s)
    }

    pub fn destroy_stream(&self, s: CUstream) {
        unsafe { ffi::lp_stream_destroy(self.ctx, s) };
    }

    /// `driver.rs:159-163` (timed, so `lp_event_elapsed_ms` works on it).
    pub fn event(&self) -> Result<CUevent> {
        let mut e = ptr::null_mut();
        check(unsafe { ffi::lp_event_create(self.ctx, &mut e) }, "lp_event_create")?;
        Ok(e)
    }

    pub fn htod_async(&self, dst: CUdeviceptr, src: &[u8], stream: CUstream) -> Result<()> {
        let rc = unsafe { ffi::lp_htod_async(self.ctx, dst, src.as_ptr() as *const c_void, src.len(), stream) };
        check(rc, "lp_htod_async")
    }

    pub fn memset_async(&self, dst: CUdeviceptr, byte: u8, len: usize, stream: CUstream) -> Result<()> {
        check(unsafe { ffi::lp_memset_async(self.ctx, dst, byte as i32, len, stream) }, "lp_memset_async")
    }

    pub fn dtoh_async(&self, dst: &mut [u8], src: CUdeviceptr, stream: CUstream) -> Result<()> {
        let rc = unsafe { ffi::lp_dtoh_async(self.ctx, dst.as_mut_ptr() as *mut c_void, src, dst.len(), stream) };
        check(rc, "lp_dtoh_async")
    }

    pub fn dtod_async(&self, dst: CUdeviceptr, src: CUdeviceptr, len: usize, stream: CUstream) -> Result<()> {
        check(unsafe { ffi::lp_dtod_async(self.ctx, dst, src, len, stream) }, "lp_dtod_async")
    }

    pub fn record_event(&self, e: CUevent, s: CUstream) -> Result<()> {
        check(unsafe { ffi::lp_record_event(self.ctx, e, s) }, "lp_record_event")
    }

    pub fn sync_event(&self, e: CUevent) -> Result<()> {
        check(unsafe { ffi::lp_sync_event(self.ctx, e) }, "lp_sync_event")
    }

    pub fn destroy_event(&self, e: CUevent) {
        unsafe { ffi::lp_event_destroy(self.ctx, e) };
    }

    /// `driver.rs:206-213`: true once the work before the event is done.
    pub fn event_done(&self, e: CUevent) -> Result<bool> {
        let rc = unsafe { ffi::lp_event_done(self.ctx, e) };
        if rc < 0 {
            check(rc, "lp_event_done")?;
        }
        Ok(rc == 1)
    }

    pub fn stream_wait_event(&self, s: CUstream, e: CUevent) -> Result<()> {
        check(unsafe { ffi::lp_stream_wait_event(self.ctx, s, e) }, "lp_stream_wait_event")
    }

    pub fn sync_stream(&self, s: CUstream) -> Result<()> {
        check(unsafe { ffi::lp_sync_stream(self.ctx, s) }, "lp_sync_stream")
    }

    pub fn sync(&self) -> Result<()> {
        check(unsafe { ffi::lp_sync(self.ctx) }, "lp_sync")
    }
}

impl Drop for Cuda {
    fn drop(&mut self) {
        unsafe { ffi::lp_destroy(self.ctx) };
    }
}

/// Page-locked host buffer (`driver.rs:286-300`); freed with
/// [`Cuda::free_pinned`], as in the reference.
pub struct Pinned {
    ptr: *mut u8,
    len: usize,
}

impl Pinned {
    pub fn as_mut(&mut self) -> &mut [u8] {
        unsafe { std::slice::from_raw_parts_mut(self.ptr, self.len) }
    }
    pub fn as_ref(&self) -> &[u8] {
        unsafe { std::slice::from_raw_parts(self.ptr, self.len) }
    }
    pub fn len(&self) -> usize {
        self.len
    }
    pub fn is_empty(&self) -> bool {
        self.len == 0
    }
}

// driver.rs:302-304: the library's context is shared across threads; every
// entry point binds its device before use.
unsafe impl Send for Pinned {}
unsafe impl Send for Cuda {}
unsafe impl Sync for Cuda {}
