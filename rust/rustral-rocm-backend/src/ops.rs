//! `TensorOps` and `AttentionOps` of the ROCm backend.
//!
//! The subset the KV path and the config-0 model need runs on the device
//! through the C ABI (`linear`, `gelu`, `add`, `argmax`, `gather_rows`, the
//! per-head attention recipe's `matmul` / `transpose` / `mul_scalar` /
//! `softmax` / `softmax_dim`, data movement for `zeros` / `slice` / `concat`
//! / `reshape`); the other methods
//! return `CoreError::Backend("<op>: unsupported on rocm backend")`.  There
//! is no host fallback.

use std::os::raw::c_void;
use std::sync::Arc;

use rustral_core::{AttentionOps, CoreError, Parameter, Result, TensorOps};

use crate::device::{Ctx, DeviceBuffer};
use crate::error::{check, hip_check, unsupported};
use crate::ffi::{self, hip};
use crate::tensor::{numel, DType, RocmTensor};
use crate::RocmBackend;

#[derive(Clone)]
pub struct RocmOps {
    pub(crate) ctx: Arc<Ctx>,
}

fn same_shape(a: &RocmTensor, b: &RocmTensor) -> Result<()> {
    if a.shape != b.shape {
        return Err(CoreError::ShapeMismatch { expected: a.shape.clone(), actual: b.shape.clone() });
    }
    Ok(())
}

fn f32_tensor(x: &RocmTensor, what: &str) -> Result<()> {
    if x.dtype != DType::F32 {
        return Err(CoreError::InvalidArgument(format!("{what}: expected an F32 tensor, got {:?}", x.dtype)));
    }
    Ok(())
}

fn to_c_int(v: usize, what: &str) -> Result<i32> {
    i32::try_from(v).map_err(|_| CoreError::InvalidArgument(format!("{what} = {v} exceeds i32")))
}

impl RocmOps {
    fn s(&self) -> ffi::Stream {
        self.ctx.stream
    }

    /// `rkv_softmax_dim` over x viewed as `[outer][axis][inner]`.
    fn softmax_lines(&self, x: &RocmTensor, outer: usize, axis: usize, inner: usize) -> Result<RocmTensor> {
        let y = RocmTensor::empty(&self.ctx, &x.shape, DType::F32)?;
        // SAFETY: x and y hold outer * axis * inner floats.
        check(unsafe {
            ffi::rkv_softmax_dim(y.device_ptr() as *mut f32, x.device_ptr() as *const f32, outer as i64,
                                 axis as i64, inner as i64, self.s())
        })?;
        Ok(y)
    }

    fn d2d(&self, dst: *mut c_void, src: *const c_void, bytes: usize) -> Result<()> {
        if bytes == 0 {
            return Ok(());
        }
        // SAFETY: both ranges lie inside live device allocations (checked by callers).
        unsafe {
            hip_check(
                hip::hipMemcpyAsync(dst, src, bytes, hip::HIP_MEMCPY_DEVICE_TO_DEVICE, self.s()),
                "hipMemcpyAsync (device to device)",
            )
        }
    }
}

impl TensorOps<RocmBackend> for RocmOps {
    fn shape(&self, x: &RocmTensor) -> Vec<usize> {
        x.shape.clone()
    }

    fn tensor_from_vec(&self, values: Vec<f32>, shape: &[usize]) -> Result<RocmTensor> {
        if values.len() != numel(shape) {
            return Err(CoreError::ShapeMismatch { expected: shape.to_vec(), actual: vec![values.len()] });
        }
        RocmTensor::upload(&self.ctx, &values, shape, DType::F32)
    }

    fn zeros(&self, shape: &[usize]) -> Result<RocmTensor> {
        let buf = DeviceBuffer::zeroed(&self.ctx, numel(shape) * 4)?;
        Ok(RocmTensor::from_buffer(&self.ctx, buf, shape, DType::F32))
    }

    /// Rank-2 product (crates/ndarray-backend/src/lib.rs:191-267) by
    /// `rkv_matmul`: every sum serial in k, the naive loop's order.
    fn matmul(&self, a: &RocmTensor, b: &RocmTensor) -> Result<RocmTensor> {
        a.expect(DType::F32, 2, "matmul a")?;
        b.expect(DType::F32, 2, "matmul b")?;
        let (m, k, n) = (a.shape[0], a.shape[1], b.shape[1]);
        if b.shape[0] != k {
            return Err(CoreError::ShapeMismatch { expected: vec![k], actual: vec![b.shape[0]] });
        }
        let y = RocmTensor::empty(&self.ctx, &[m, n], DType::F32)?;
        // SAFETY: a [m][k], b [k][n] and y [m][n] are live device buffers.
        check(unsafe {
            ffi::rkv_matmul(y.device_ptr() as *mut f32, a.device_ptr() as *const f32, b.device_ptr() as *const f32,
                            to_c_int(m, "m")?, to_c_int(k, "k")?, to_c_int(n, "n")?, self.s())
        })?;
        Ok(y)
    }

    /// Rank-2 transpose (lib.rs:270-281) by `rkv_transpose`.
    fn transpose(&self, x: &RocmTensor) -> Result<RocmTensor> {
        x.expect(DType::F32, 2, "transpose")?;
        let (m, n) = (x.shape[0], x.shape[1]);
        let y = RocmTensor::empty(&self.ctx, &[n, m], DType::F32)?;
        // SAFETY: x [m][n] and y [n][m] are distinct live device buffers.
        check(unsafe {
            ffi::rkv_transpose(y.device_ptr() as *mut f32, x.device_ptr() as *const f32, to_c_int(m, "m")?,
                               to_c_int(n, "n")?, self.s())
        })?;
        Ok(y)
    }

    /// Element-wise sum (crates/ndarray-backend/src/lib.rs:283-315) by `rkv_add`.
    fn add(&self, a: &RocmTensor, b: &RocmTensor) -> Result<RocmTensor> {
        f32_tensor(a, "add")?;
        f32_tensor(b, "add")?;
        same_shape(a, b)?;
        let y = RocmTensor::empty(&self.ctx, &a.shape, DType::F32)?;
        // SAFETY: three live device buffers of numel floats each.
        check(unsafe {
            ffi::rkv_add(y.device_ptr() as *mut f32, a.device_ptr() as *const f32,
                         b.device_ptr() as *const f32, a.numel() as i64, self.s())
        })?;
        Ok(y)
    }

    fn add_row_vector(&self, _a: &RocmTensor, _row: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("add_row_vector"))
    }

    fn relu(&self, _x: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("relu"))
    }

    /// Softmax over all values (lib.rs:373-427) as one line of
    /// `rkv_softmax_dim`; the reference's `wide` SIMD exp is not reproduced
    /// (the device expf is within 2 ulp of the host's).
    fn softmax(&self, x: &RocmTensor) -> Result<RocmTensor> {
        f32_tensor(x, "softmax")?;
        if x.numel() == 0 {
            return Err(CoreError::InvalidArgument("softmax of empty tensor".into()));
        }
        self.softmax_lines(x, 1, x.numel(), 1)
    }

    /// Softmax along `dim` (lib.rs:1188-1227) by `rkv_softmax_dim`: per line
    /// max, `exp(x - max)`, the serial sum and `* (1 / sum)`.
    fn softmax_dim(&self, x: &RocmTensor, dim: usize) -> Result<RocmTensor> {
        f32_tensor(x, "softmax_dim")?;
        if dim >= x.shape.len() {
            return Err(CoreError::InvalidArgument(format!(
                "softmax_dim: dim {dim} out of range for shape {:?}", x.shape
            )));
        }
        let axis = x.shape[dim];
        if axis == 0 {
            return Err(CoreError::InvalidArgument("softmax_dim: axis size is 0".into()));
        }
        self.softmax_lines(x, numel(&x.shape[..dim]), axis, numel(&x.shape[dim + 1..]))
    }

    fn log_softmax(&self, _x: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("log_softmax"))
    }

    /// Flat index of the largest value, the last one on ties (`max_by`,
    /// crates/ndarray-backend/src/lib.rs:430-437), by `rkv_argmax`.
    fn argmax(&self, x: &RocmTensor) -> Result<usize> {
        f32_tensor(x, "argmax")?;
        let n = to_c_int(x.numel(), "argmax length")?;
        if n == 0 {
            return Err(CoreError::InvalidArgument("argmax of an empty tensor".into()));
        }
        let out = RocmTensor::empty(&self.ctx, &[1], DType::I32)?;
        // SAFETY: x holds n floats, out one int32.
        check(unsafe { ffi::rkv_argmax(out.device_ptr() as *mut i32, x.device_ptr() as *const f32, 1, n, self.s()) })?;
        let v = out.to_vec_i32()?;
        Ok(v[0] as usize)
    }

    /// Rows of an embedding table (crates/ndarray-backend/src/lib.rs:462-475)
    /// by `rkv_embed` without a positional table; an id outside the table
    /// gives a NaN row, as the kernel documents.
    fn gather_rows(&self, table: &Parameter<RocmBackend>, ids: &[usize]) -> Result<RocmTensor> {
        let t = table.tensor();
        t.expect(DType::F32, 2, "gather_rows table")?;
        let (vocab, dim) = (t.shape[0], t.shape[1]);
        let ids32: Vec<i32> = ids.iter().map(|&i| i32::try_from(i).unwrap_or(-1)).collect();
        let dids = RocmTensor::upload(&self.ctx, &ids32, &[ids.len()], DType::I32)?;
        let y = RocmTensor::empty(&self.ctx, &[ids.len(), dim], DType::F32)?;
        // SAFETY: table [vocab][dim], ids [n], y [n][dim] are live device buffers.
        check(unsafe {
            ffi::rkv_embed(y.device_ptr() as *mut f32, t.device_ptr() as *const f32,
                           dids.device_ptr() as *const i32, std::ptr::null(), std::ptr::null(),
                           to_c_int(ids.len(), "ids")?, to_c_int(vocab, "vocab")?, to_c_int(dim, "dim")?,
                           0, self.s())
        })?;
        Ok(y)
    }

    /// `input * weight^T + bias` with the reference's serial sums
    /// (crates/ndarray-backend/src/lib.rs:478-534) by `rkv_linear`.
    fn linear(
        &self,
        input: &RocmTensor,
        weight: &Parameter<RocmBackend>,
        bias: Option<&Parameter<RocmBackend>>,
    ) -> Result<RocmTensor> {
        f32_tensor(input, "linear input")?;
        let w = weight.tensor();
        w.expect(DType::F32, 2, "linear weight")?;
        let (out_dim, in_dim) = (w.shape[0], w.shape[1]);
        let (rows, out_shape) = match input.shape.as_slice() {
            [k] if *k == in_dim => (1usize, vec![out_dim]),
            [r, k] if *k == in_dim => (*r, vec![*r, out_dim]),
            _ => {
                return Err(CoreError::ShapeMismatch { expected: vec![in_dim], actual: input.shape.clone() })
            }
        };
        let b_ptr = match bias {
            Some(b) => {
                b.tensor().expect(DType::F32, 1, "linear bias")?;
                if b.tensor().shape[0] != out_dim {
                    return Err(CoreError::ShapeMismatch { expected: vec![out_dim], actual: b.tensor().shape.clone() });
                }
                b.tensor().device_ptr() as *const f32
            }
            None => std::ptr::null(),
        };
        let y = RocmTensor::empty(&self.ctx, &out_shape, DType::F32)?;
        // SAFETY: x [rows][in], w [out][in], b [out] or NULL, y [rows][out].
        check(unsafe {
            ffi::rkv_linear(y.device_ptr() as *mut f32, input.device_ptr() as *const f32,
                            w.device_ptr() as *const f32, b_ptr, to_c_int(rows, "rows")?,
                            to_c_int(in_dim, "in_dim")?, to_c_int(out_dim, "out_dim")?, self.s())
        })?;
        Ok(y)
    }

    fn sigmoid(&self, _x: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("sigmoid"))
    }

    fn tanh(&self, _x: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("tanh"))
    }

    /// tanh-approximated GELU (crates/ndarray-backend/src/lib.rs:565-598) by `rkv_gelu`.
    fn gelu(&self, x: &RocmTensor) -> Result<RocmTensor> {
        f32_tensor(x, "gelu")?;
        let y = RocmTensor::empty(&self.ctx, &x.shape, DType::F32)?;
        // SAFETY: x and y hold numel floats.
        check(unsafe {
            ffi::rkv_gelu(y.device_ptr() as *mut f32, x.device_ptr() as *const f32, x.numel() as i64, self.s())
        })?;
        Ok(y)
    }

    fn mul(&self, _a: &RocmTensor, _b: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("mul"))
    }

    /// Inference (training = false) is the identity, as the reference
    /// defines it; training-mode dropout is not built.
    fn dropout(&self, x: &RocmTensor, _p: f32, training: bool) -> Result<RocmTensor> {
        if training {
            return Err(unsupported("dropout (training)"));
        }
        Ok(x.clone())
    }

    /// Concatenation along dimension 0 by device-to-device copies.
    fn concat(&self, tensors: &[&RocmTensor], dim: usize) -> Result<RocmTensor> {
        if dim != 0 || tensors.is_empty() {
            return Err(unsupported("concat (only along dimension 0)"));
        }
        if let Some(t) = tensors.iter().find(|t| t.shape.is_empty()) {
            return Err(CoreError::InvalidArgument(format!("concat: rank-0 tensor {:?}", t.shape)));
        }
        let first = tensors[0];
        let tail = &first.shape[1..];
        let mut rows = 0usize;
        for t in tensors {
            if t.dtype != first.dtype || &t.shape[1..] != tail {
                return Err(CoreError::ShapeMismatch { expected: first.shape.clone(), actual: t.shape.clone() });
            }
            rows += t.shape[0];
        }
        let mut shape = vec![rows];
        shape.extend_from_slice(tail);
        let y = RocmTensor::empty(&self.ctx, &shape, first.dtype)?;
        let mut off = 0usize;
        for t in tensors {
            let bytes = t.numel() * t.dtype.size();
            // SAFETY: destination range [off, off + bytes) lies inside y.
            let dst = unsafe { (y.device_ptr() as *mut u8).add(off) } as *mut c_void;
            self.d2d(dst, t.device_ptr(), bytes)?;
            off += bytes;
        }
        Ok(y)
    }

    /// Rows start..end of dimension 0 (a device-to-device copy).
    fn slice(&self, x: &RocmTensor, start: usize, end: usize) -> Result<RocmTensor> {
        if x.shape.is_empty() || start > end || end > x.shape[0] {
            return Err(CoreError::InvalidArgument(format!("slice {start}..{end} of {:?}", x.shape)));
        }
        let row = x.numel() / x.shape[0].max(1) * x.dtype.size();
        let mut shape = x.shape.clone();
        shape[0] = end - start;
        let y = RocmTensor::empty(&self.ctx, &shape, x.dtype)?;
        // SAFETY: rows start..end lie inside x.
        let src = unsafe { (x.device_ptr() as *const u8).add(start * row) } as *const c_void;
        self.d2d(y.device_ptr(), src, (end - start) * row)?;
        Ok(y)
    }

    fn reshape(&self, x: &RocmTensor, shape: &[usize]) -> Result<RocmTensor> {
        x.reshaped(shape)
    }

    fn add_scalar(&self, _x: &RocmTensor, _s: f32) -> Result<RocmTensor> {
        Err(unsupported("add_scalar"))
    }

    /// `x * s` per element (lib.rs:747-756) by `rkv_mul_scalar`.
    fn mul_scalar(&self, x: &RocmTensor, s: f32) -> Result<RocmTensor> {
        f32_tensor(x, "mul_scalar")?;
        let y = RocmTensor::empty(&self.ctx, &x.shape, DType::F32)?;
        // SAFETY: x and y hold numel floats.
        check(unsafe {
            ffi::rkv_mul_scalar(y.device_ptr() as *mut f32, x.device_ptr() as *const f32, s, x.numel() as i64,
                                self.s())
        })?;
        Ok(y)
    }

    fn broadcast(&self, _x: &RocmTensor, _shape: &[usize]) -> Result<RocmTensor> {
        Err(unsupported("broadcast"))
    }

    fn neg(&self, _x: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("neg"))
    }

    fn sub(&self, _a: &RocmTensor, _b: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("sub"))
    }

    fn sqrt(&self, _x: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("sqrt"))
    }

    fn div(&self, _a: &RocmTensor, _b: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("div"))
    }

    fn exp(&self, _x: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("exp"))
    }

    fn log(&self, _x: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("log"))
    }

    fn maximum(&self, _a: &RocmTensor, _b: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("maximum"))
    }

    fn gt_scalar(&self, _x: &RocmTensor, _s: f32) -> Result<RocmTensor> {
        Err(unsupported("gt_scalar"))
    }

    fn sum_all(&self, _x: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("sum_all"))
    }

    fn sum_dim0(&self, _x: &RocmTensor) -> Result<RocmTensor> {
        Err(unsupported("sum_dim0"))
    }

    fn tensor_to_vec(&self, x: &RocmTensor) -> Result<Vec<f32>> {
        x.to_vec_f32()
    }

    fn tensor_element(&self, x: &RocmTensor, index: usize) -> Result<f32> {
        if index >= x.numel() {
            return Err(CoreError::InvalidArgument(format!("index {index} of {} elements", x.numel())));
        }
        Ok(self.slice(&x.reshaped(&[x.numel()])?, index, index + 1)?.to_vec_f32()?[0])
    }
}

/// Causal attention over dense `[batch, seq, heads, head_dim]` tensors
/// (crates/core/src/backend.rs:551-602) on the paged prefill kernel: K and V
/// are appended into a temporary pool (`ceil(seq / 16)` blocks per batch
/// entry, identity tables) and `rkv_prefill_attention` runs every query row
/// against positions `0..=row` with scale `1 / sqrt(head_dim)`.  Non-causal
/// and masked attention are not built.
impl AttentionOps<RocmBackend> for RocmOps {
    fn flash_attention_2(
        &self,
        query: &RocmTensor,
        key: &RocmTensor,
        value: &RocmTensor,
        causal_mask: bool,
    ) -> Result<RocmTensor> {
        if !causal_mask {
            return Err(unsupported("flash_attention_2 (non-causal)"));
        }
        for (t, n) in [(query, "query"), (key, "key"), (value, "value")] {
            t.expect(DType::F32, 4, n)?;
        }
        same_shape(query, key)?;
        same_shape(query, value)?;
        let (b, s, h, d) = (query.shape[0], query.shape[1], query.shape[2], query.shape[3]);
        let nblk = (s + 15) / 16;
        let pool_elems = b * nblk * h * 16 * d;
        let kp = DeviceBuffer::new(pool_elems * 4)?;
        let vp = DeviceBuffer::new(pool_elems * 4)?;
        let slots: Vec<i64> = (0..b).flat_map(|bi| (0..s).map(move |t| (bi * nblk * 16 + t) as i64)).collect();
        let tables: Vec<i32> = (0..b * nblk).map(|i| i as i32).collect();
        let q_start: Vec<i32> = (0..=b).map(|bi| (bi * s) as i32).collect();
        let lens = vec![s as i32; b];
        let dslots = RocmTensor::upload(&self.ctx, &slots, &[b * s], DType::I64)?;
        let dtab = RocmTensor::upload(&self.ctx, &tables, &[b, nblk], DType::I32)?;
        let dq0 = RocmTensor::upload(&self.ctx, &q_start, &[b + 1], DType::I32)?;
        let dlen = RocmTensor::upload(&self.ctx, &lens, &[b], DType::I32)?;
        let (ci, cd, ch) = (to_c_int(b, "batch")?, to_c_int(d, "head_dim")?, to_c_int(h, "heads")?);
        let tok_stride = (h * d) as i64;
        // SAFETY: every pointer is a live device buffer of the documented size.
        unsafe {
            check(ffi::rkv_append(kp.ptr(), vp.ptr(), 0, key.device_ptr() as *const f32,
                                  value.device_ptr() as *const f32, 0, tok_stride, d as i64,
                                  dslots.device_ptr() as *const i64, (b * s) as i64, 1, ch, cd, 16,
                                  (b * nblk) as i64, ffi::RKV_F32, self.s()))?;
        }
        let out = RocmTensor::empty(&self.ctx, &query.shape, DType::F32)?;
        // SAFETY: as above; q and out are [b*s][h][d].
        unsafe {
            check(ffi::rkv_prefill_attention(out.device_ptr() as *mut f32, query.device_ptr() as *const f32,
                                             kp.ptr(), vp.ptr(), dtab.device_ptr() as *const i32,
                                             to_c_int(nblk, "blocks")?, dq0.device_ptr() as *const i32,
                                             dlen.device_ptr() as *const i32, ci, ch, ch, cd, 16,
                                             (b * nblk) as i64, to_c_int(s, "seq")?,
                                             1.0 / (d as f32).sqrt(), ffi::RKV_F32, self.s()))?;
        }
        // the temporary pools are freed after the stream has used them
        self.ctx.synchronize()?;
        Ok(out)
    }

    fn flash_attention_2_with_mask(
        &self,
        _query: &RocmTensor,
        _key: &RocmTensor,
        _value: &RocmTensor,
        _mask: &RocmTensor,
    ) -> Result<RocmTensor> {
        Err(unsupported("flash_attention_2_with_mask"))
    }
}
