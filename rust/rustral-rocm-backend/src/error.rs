//! Status codes of the C ABI and HIP runtime errors as `CoreError`s.

use std::ffi::CStr;
use std::os::raw::c_int;

use rustral_core::{CoreError, Result};

use crate::ffi;

/// The library's thread-local message for the last failing call.
pub fn last_error() -> String {
    // SAFETY: rkv_last_error returns a pointer to a thread-local NUL-terminated
    // string owned by the library, valid until the next call on this thread.
    unsafe {
        let p = ffi::rkv_last_error();
        if p.is_null() {
            String::new()
        } else {
            CStr::from_ptr(p).to_string_lossy().into_owned()
        }
    }
}

/// Maps a C-ABI status to `CoreError` with the library's message, as the
/// candle backend maps its errors (crates/candle-backend/src/lib.rs:300-312):
/// invalid arguments and shapes to `InvalidArgument`, an exhausted KV pool to
/// `Other` (what `Scheduler::update` reports, continuous_batching.rs:315),
/// everything else (unsupported shape, workspace, HIP failure) to `Backend`.
/// Nothing panics across the FFI boundary.
pub fn check(rc: c_int) -> Result<()> {
    if rc == ffi::RKV_OK {
        return Ok(());
    }
    let msg = last_error();
    Err(match rc {
        ffi::RKV_ERR_INVALID_ARG => CoreError::InvalidArgument(msg),
        ffi::RKV_ERR_OOM => CoreError::Other(msg),
        _ => CoreError::Backend(msg),
    })
}

/// A HIP runtime status as `CoreError::Backend`.
pub fn hip_check(e: ffi::hip::HipError, what: &str) -> Result<()> {
    if e == ffi::hip::HIP_SUCCESS {
        return Ok(());
    }
    // SAFETY: hipGetErrorString returns a static NUL-terminated string.
    let s = unsafe {
        let p = ffi::hip::hipGetErrorString(e);
        if p.is_null() {
            format!("HIP error {e}")
        } else {
            CStr::from_ptr(p).to_string_lossy().into_owned()
        }
    };
    Err(CoreError::Backend(format!("{what}: {s}")))
}

/// The error every `TensorOps` method this backend leaves out returns (the
/// pattern of the wgpu backend for its missing ops,
/// crates/wgpu-backend/src/lib.rs:1477-1483).
pub fn unsupported(op: &str) -> CoreError {
    CoreError::Backend(format!("{op}: unsupported on rocm backend"))
}
