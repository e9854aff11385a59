//! The ROCm backend of rustral for MI355X (gfx950): rustral's paged KV-cache
//! hot path -- per-layer K/V append into a block-paged cache, gathers through
//! block tables, block copy for compaction, and GQA decode / causal prefill
//! attention over the paged cache -- on hand-written HIP kernels behind the C
//! ABI of librustral_kv (include/*.h; `build.rs` compiles the kernels with
//! hipcc for gfx950).
//!
//! * [`RocmBackend`] implements `Backend` (crates/core/src/backend.rs:140-205):
//!   one HIP stream per instance, device tensors ([`RocmTensor`]) that satisfy
//!   the bound the reference's `KVCache<B>` / `PagedCache<B>` / `Scheduler<B>`
//!   put on `B::Tensor` (`Clone + AsRef<[f32]> + TensorShape`,
//!   crates/nn/src/kv_cache.rs:154-157), so generic rustral code compiles
//!   against it unchanged.
//! * [`RocmOps`] implements `TensorOps` (:212-399) for the subset the path
//!   and the config-0 model use, and `AttentionOps` (:551-602) for causal
//!   attention; every other op returns `CoreError::Backend`.
//! * [`RocmPagedKvCache`] is the paged API the serving loop calls: it takes
//!   the scheduler's `Batch.block_tables` / `seq_lens` (converted once per
//!   step by [`batch_to_device`]).
//! * [`BlockManager`] / [`DeviceBlockManager`] are `PagedCache` on the host
//!   and in device memory.
//! * [`RocmDecoder`] runs the config-0 decoder end to end (greedy
//!   `generate_token`, crates/nn/src/transformer.rs:837-862) and
//!   [`RocmServingEngine`] is `ServingEngine` (crates/nn/src/
//!   continuous_batching.rs:493-545) with the model in its step.

pub mod ffi;

mod device;
mod error;
mod model;
mod ops;
mod paged;
mod serving;
mod tensor;

use std::sync::Arc;

use rustral_core::{AttentionOps, Backend, BackendCapabilities, CoreError, Parameter, Result, TensorOps, TrainingDtype};

pub use device::{Ctx, DeviceBuffer};
pub use error::{check, last_error};
pub use model::{DecoderConfig, Priority, RocmDecoder, RocmServingEngine, SchedulerStats};
pub use ops::RocmOps;
pub use paged::{batch_to_device, KvDtype, PagedKvConfig, RocmPagedKvCache, BLOCK_SIZE};
pub use serving::{BlockManager, DeviceBlockManager};
pub use tensor::{DType, RocmTensor};

/// A GPU by ordinal.
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub struct RocmDevice {
    pub ordinal: i32,
}

/// The backend: a device and its stream, shared by clones.
#[derive(Clone)]
pub struct RocmBackend {
    pub(crate) ctx: Arc<Ctx>,
    ops: RocmOps,
}

impl RocmBackend {
    /// A backend on GPU `ordinal` with a stream of its own.
    pub fn new(ordinal: i32) -> Result<Self> {
        let ctx = Arc::new(Ctx::new(ordinal)?);
        Ok(Self { ops: RocmOps { ctx: ctx.clone() }, ctx })
    }

    /// Waits for every launch enqueued by this backend.
    pub fn synchronize(&self) -> Result<()> {
        self.ctx.synchronize()
    }

    /// A device int32 tensor (block tables, lengths, ids).
    pub fn tensor_from_i32(&self, values: &[i32], shape: &[usize]) -> Result<RocmTensor> {
        RocmTensor::upload(&self.ctx, values, shape, DType::I32)
    }

    /// A device int64 tensor (slot mappings).
    pub fn tensor_from_i64(&self, values: &[i64], shape: &[usize]) -> Result<RocmTensor> {
        RocmTensor::upload(&self.ctx, values, shape, DType::I64)
    }

    /// Named parameters from a safetensors file with the reference's strict
    /// `load_model` rules (crates/runtime/src/model_io.rs:36-105: missing or
    /// extra keys, a shape mismatch, a dtype other than F32 are errors),
    /// copied straight from the memory-mapped file into device tensors.
    pub fn load_safetensors(&self, path: &str, wanted: &[(&str, &[usize])]) -> Result<Vec<Parameter<Self>>> {
        let cpath = std::ffi::CString::new(path).map_err(|e| CoreError::InvalidArgument(e.to_string()))?;
        // SAFETY: NUL-terminated path.
        let f = unsafe { ffi::rkv_st_open(cpath.as_ptr()) };
        if f.is_null() {
            return Err(CoreError::Serialization(last_error()));
        }
        let result: Result<Vec<Parameter<Self>>> = (|| {
            let tensors: Vec<RocmTensor> = wanted
                .iter()
                .map(|(_, shape)| RocmTensor::empty(&self.ctx, shape, DType::F32))
                .collect::<Result<_>>()?;
            let names: Vec<std::ffi::CString> = wanted
                .iter()
                .map(|(n, _)| std::ffi::CString::new(*n).map_err(|e| CoreError::InvalidArgument(e.to_string())))
                .collect::<Result<_>>()?;
            let name_ptrs: Vec<*const std::os::raw::c_char> = names.iter().map(|n| n.as_ptr()).collect();
            let ndims: Vec<i32> = wanted.iter().map(|(_, s)| s.len() as i32).collect();
            let shapes: Vec<i64> = wanted.iter().flat_map(|(_, s)| s.iter().map(|&d| d as i64)).collect();
            let dsts: Vec<*mut std::os::raw::c_void> = tensors.iter().map(|t| t.device_ptr()).collect();
            // SAFETY: every array holds wanted.len() entries (shapes: the sum of ndims).
            let rc = unsafe {
                ffi::rkv_st_load(f, wanted.len() as i32, name_ptrs.as_ptr(), ndims.as_ptr(), shapes.as_ptr(),
                                 dsts.as_ptr(), 1, self.ctx.stream)
            };
            if rc != ffi::RKV_OK {
                return Err(CoreError::Serialization(last_error()));
            }
            Ok(wanted.iter().zip(tensors).map(|((n, _), t)| Parameter::new(*n, t)).collect())
        })();
        // SAFETY: opened above, closed once.
        unsafe { ffi::rkv_st_close(f) };
        result
    }
}

impl Backend for RocmBackend {
    type Tensor = RocmTensor;
    type Device = RocmDevice;

    fn device(&self) -> RocmDevice {
        RocmDevice { ordinal: self.ctx.device }
    }

    fn ops(&self) -> &dyn TensorOps<Self> {
        &self.ops
    }

    fn attention_ops(&self) -> Option<&dyn AttentionOps<Self>> {
        Some(&self.ops)
    }

    fn capabilities(&self) -> BackendCapabilities {
        BackendCapabilities {
            supports_bf16: true,
            tensor_cores: true,
            optimal_batch_size: 64,
            recommended_training_dtype: TrainingDtype::F32,
            ..BackendCapabilities::default()
        }
    }

    fn as_any(&self) -> &dyn std::any::Any {
        self
    }

    /// Uniform values in `[-scale, scale)` (zeros for `scale <= 0`), as the
    /// reference's `normal_parameter` documents (crates/ndarray-backend/src/
    /// lib.rs:132-146), drawn from this library's PCG64 stream
    /// (`rkv_rng_raw`, seeded with `seed`): `u = (x >> 11) * 2^-53`, value
    /// `(2u - 1) * scale`.  The reference's ChaCha12 `StdRng` stream is not
    /// reproduced.
    fn normal_parameter(&self, name: &str, shape: &[usize], seed: u64, scale: f32) -> Result<Parameter<Self>> {
        let n: usize = shape.iter().product();
        let values = if scale <= 0.0 {
            vec![0f32; n]
        } else {
            let mut raw = vec![0u64; n];
            // SAFETY: raw holds n entries.
            check(unsafe { ffi::rkv_rng_raw(seed, raw.as_mut_ptr(), n as i64) })?;
            raw.into_iter()
                .map(|x| ((2.0 * (x >> 11) as f64 * (1.0 / 9007199254740992.0) - 1.0) * scale as f64) as f32)
                .collect()
        };
        self.parameter_from_vec(name, values, shape)
    }

    fn parameter_from_vec(&self, name: &str, values: Vec<f32>, shape: &[usize]) -> Result<Parameter<Self>> {
        Ok(Parameter::new(name, self.ops.tensor_from_vec(values, shape)?))
    }
}
