//! `RocmTensor`: a shaped view of a device buffer.

use std::sync::{Arc, OnceLock};

use rustral_core::{CoreError, Result, TensorShape};

use crate::device::{Ctx, DeviceBuffer};

/// Element type of a device tensor.  Model tensors are `F32`; `Bf16` holds
/// gathered 16-bit KV rows; `I32` / `I64` hold block tables, lengths, ids and
/// slot mappings for the paged calls.
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum DType {
    F32,
    Bf16,
    I32,
    I64,
}

impl DType {
    pub fn size(self) -> usize {
        match self {
            DType::F32 | DType::I32 => 4,
            DType::Bf16 => 2,
            DType::I64 => 8,
        }
    }
}

/// A device tensor.  Tensors are values, as `TensorOps` is functional
/// (crates/core/src/backend.rs:212-399): every op returns a new tensor and a
/// tensor's bytes never change after it has been produced, so clones share
/// the buffer.
///
/// The reference's `KVCache<B>` and `TransformerDecoder<B>` require
/// `B::Tensor: AsRef<[f32]>` (crates/nn/src/kv_cache.rs:154-157).  For code
/// under that bound the tensor keeps a host mirror, filled on the first
/// `as_ref()` by one synchronous device-to-host copy (a `Bf16` tensor is
/// widened exactly; integer tensors and failed copies give an empty slice,
/// since the trait has no error channel).  The paged API never uses it.
#[derive(Clone)]
pub struct RocmTensor {
    pub(crate) buf: Arc<DeviceBuffer>,
    pub(crate) shape: Vec<usize>,
    pub(crate) dtype: DType,
    pub(crate) ctx: Arc<Ctx>,
    mirror: Arc<OnceLock<Vec<f32>>>,
}

impl std::fmt::Debug for RocmTensor {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        f.debug_struct("RocmTensor").field("shape", &self.shape).field("dtype", &self.dtype).finish()
    }
}

pub(crate) fn numel(shape: &[usize]) -> usize {
    shape.iter().product()
}

impl RocmTensor {
    pub(crate) fn from_buffer(ctx: &Arc<Ctx>, buf: DeviceBuffer, shape: &[usize], dtype: DType) -> Self {
        Self {
            buf: Arc::new(buf),
            shape: shape.to_vec(),
            dtype,
            ctx: ctx.clone(),
            mirror: Arc::new(OnceLock::new()),
        }
    }

    /// An uninitialised tensor for a call's output.
    pub(crate) fn empty(ctx: &Arc<Ctx>, shape: &[usize], dtype: DType) -> Result<Self> {
        let buf = DeviceBuffer::new(numel(shape) * dtype.size())?;
        Ok(Self::from_buffer(ctx, buf, shape, dtype))
    }

    pub(crate) fn upload<T: Copy>(ctx: &Arc<Ctx>, data: &[T], shape: &[usize], dtype: DType) -> Result<Self> {
        if std::mem::size_of::<T>() != dtype.size() || data.len() != numel(shape) {
            return Err(CoreError::ShapeMismatch { expected: vec![numel(shape)], actual: vec![data.len()] });
        }
        let t = Self::empty(ctx, shape, dtype)?;
        t.buf.upload(ctx, data)?;
        Ok(t)
    }

    pub fn dtype(&self) -> DType {
        self.dtype
    }

    pub fn numel(&self) -> usize {
        numel(&self.shape)
    }

    /// The device address (for the C ABI).
    pub fn device_ptr(&self) -> *mut std::os::raw::c_void {
        self.buf.ptr()
    }

    /// The same bytes under another shape of equal element count.
    pub fn reshaped(&self, shape: &[usize]) -> Result<Self> {
        if numel(shape) != self.numel() {
            return Err(CoreError::ShapeMismatch { expected: self.shape.clone(), actual: shape.to_vec() });
        }
        let mut t = self.clone();
        t.shape = shape.to_vec();
        t.mirror = Arc::new(OnceLock::new());
        Ok(t)
    }

    /// Synchronous copy of an `F32` or `Bf16` tensor to the host as f32.
    pub fn to_vec_f32(&self) -> Result<Vec<f32>> {
        match self.dtype {
            DType::F32 => {
                let mut v = vec![0f32; self.numel()];
                self.buf.download(&self.ctx, &mut v)?;
                Ok(v)
            }
            DType::Bf16 => {
                let mut v = vec![0u16; self.numel()];
                self.buf.download(&self.ctx, &mut v)?;
                Ok(v.into_iter().map(|b| f32::from_bits((b as u32) << 16)).collect())
            }
            _ => Err(CoreError::InvalidArgument(format!("tensor of {:?} is not a float tensor", self.dtype))),
        }
    }

    /// Synchronous copy of an `I32` tensor to the host.
    pub fn to_vec_i32(&self) -> Result<Vec<i32>> {
        if self.dtype != DType::I32 {
            return Err(CoreError::InvalidArgument("not an I32 tensor".into()));
        }
        let mut v = vec![0i32; self.numel()];
        self.buf.download(&self.ctx, &mut v)?;
        Ok(v)
    }

    pub(crate) fn expect(&self, dtype: DType, rank: usize, what: &str) -> Result<()> {
        if self.dtype != dtype || self.shape.len() != rank {
            return Err(CoreError::InvalidArgument(format!(
                "{what}: expected a rank-{rank} {dtype:?} tensor, got {:?} {:?}",
                self.dtype, self.shape
            )));
        }
        Ok(())
    }
}

impl AsRef<[f32]> for RocmTensor {
    fn as_ref(&self) -> &[f32] {
        self.mirror.get_or_init(|| self.to_vec_f32().unwrap_or_default()).as_slice()
    }
}

impl TensorShape for RocmTensor {
    fn shape(&self) -> &[usize] {
        &self.shape
    }
}
