//! Device memory and the backend's stream.

use std::os::raw::c_void;
use std::ptr;

use rustral_core::Result;

use crate::error::hip_check;
use crate::ffi::{self, hip};

/// One HIP stream per backend instance; every call of the backend enqueues
/// its launches on it in order.  Created non-blocking with the default
/// priority.
pub struct Ctx {
    pub(crate) device: i32,
    pub(crate) stream: ffi::Stream,
}

// SAFETY: a hipStream_t may be used from any host thread; the library's calls
// are reentrant (its only global state is the thread-local last error).
unsafe impl Send for Ctx {}
unsafe impl Sync for Ctx {}

impl Ctx {
    pub fn new(device: i32) -> Result<Self> {
        // SAFETY: plain HIP runtime calls with valid out-pointers.
        unsafe {
            hip_check(hip::hipSetDevice(device), "hipSetDevice")?;
            let mut s: *mut c_void = ptr::null_mut();
            hip_check(
                hip::hipStreamCreateWithFlags(&mut s, hip::HIP_STREAM_NON_BLOCKING),
                "hipStreamCreateWithFlags",
            )?;
            Ok(Self { device, stream: s })
        }
    }

    /// Waits for everything enqueued so far.
    pub fn synchronize(&self) -> Result<()> {
        // SAFETY: the stream is owned by self and alive.
        unsafe { hip_check(hip::hipStreamSynchronize(self.stream), "hipStreamSynchronize") }
    }
}

impl Drop for Ctx {
    fn drop(&mut self) {
        // SAFETY: the stream was created by Ctx::new and is destroyed once.
        unsafe {
            let _ = hip::hipStreamSynchronize(self.stream);
            let _ = hip::hipStreamDestroy(self.stream);
        }
    }
}

/// An owned device allocation, freed on drop.  The C ABI never frees caller
/// memory: buffers belong to the Rust side.
pub struct DeviceBuffer {
    ptr: *mut c_void,
    bytes: usize,
}

// SAFETY: the allocation is plain device memory; access is ordered by the
// backend's stream.
unsafe impl Send for DeviceBuffer {}
unsafe impl Sync for DeviceBuffer {}

impl DeviceBuffer {
    pub fn new(bytes: usize) -> Result<Self> {
        let mut p: *mut c_void = ptr::null_mut();
        if bytes > 0 {
            // SAFETY: valid out-pointer; size > 0.
            unsafe { hip_check(hip::hipMalloc(&mut p, bytes), "hipMalloc")? };
        }
        Ok(Self { ptr: p, bytes })
    }

    /// A zero-filled allocation (stream-ordered fill on `ctx`).
    pub fn zeroed(ctx: &Ctx, bytes: usize) -> Result<Self> {
        let b = Self::new(bytes)?;
        if bytes > 0 {
            // SAFETY: the range is inside the allocation.
            unsafe { hip_check(hip::hipMemsetAsync(b.ptr, 0, bytes, ctx.stream), "hipMemsetAsync")? };
        }
        Ok(b)
    }

    pub fn ptr(&self) -> *mut c_void {
        self.ptr
    }

    pub fn bytes(&self) -> usize {
        self.bytes
    }

    /// Stream-ordered upload of `src` into the start of the buffer.
    pub fn upload<T: Copy>(&self, ctx: &Ctx, src: &[T]) -> Result<()> {
        let n = std::mem::size_of_val(src);
        assert!(n <= self.bytes, "upload larger than the buffer");
        if n == 0 {
            return Ok(());
        }
        // SAFETY: src is a live host slice of n bytes; the destination holds n bytes.
        // The copy completes before the stream runs anything enqueued later, and
        // the synchronize below keeps `src` alive until then.
        unsafe {
            hip_check(
                hip::hipMemcpyAsync(
                    self.ptr,
                    src.as_ptr() as *const c_void,
                    n,
                    hip::HIP_MEMCPY_HOST_TO_DEVICE,
                    ctx.stream,
                ),
                "hipMemcpyAsync (upload)",
            )?;
        }
        ctx.synchronize()
    }

    /// Waits for the stream, then copies the first `dst.len()` elements back.
    pub fn download<T: Copy>(&self, ctx: &Ctx, dst: &mut [T]) -> Result<()> {
        let n = std::mem::size_of_val(dst);
        assert!(n <= self.bytes, "download larger than the buffer");
        if n == 0 {
            return Ok(());
        }
        // SAFETY: dst is a live host slice of n bytes; the source holds n bytes.
        unsafe {
            hip_check(
                hip::hipMemcpyAsync(
                    dst.as_mut_ptr() as *mut c_void,
                    self.ptr,
                    n,
                    hip::HIP_MEMCPY_DEVICE_TO_HOST,
                    ctx.stream,
                ),
                "hipMemcpyAsync (download)",
            )?;
        }
        ctx.synchronize()
    }
}

impl Drop for DeviceBuffer {
    fn drop(&mut self) {
        if !self.ptr.is_null() {
            // SAFETY: allocated by hipMalloc in DeviceBuffer::new, freed once.
            unsafe {
                let _ = hip::hipFree(self.ptr);
            }
        }
    }
}
