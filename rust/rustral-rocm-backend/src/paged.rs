//! `RocmPagedKvCache`: the paged KV pools of every layer and the hot-path
//! calls over them (append, gather, block copy, decode and prefill
//! attention).
//!
//! Layout: per layer and per K/V, `[num_blocks][Hkv][16][head_dim]` in one
//! allocation of all layers (layer stride `num_blocks * Hkv * 16 * head_dim`
//! elements); a sequence's token p lives in row `p % 16` of block
//! `block_table[p / 16]`.  1-byte pools (`CacheQuantization::{Int8, Fp8}`)
//! add an fp32 scale per (block, head, row).

use std::os::raw::c_void;
use std::sync::{Arc, Mutex};

use rustral_core::{CoreError, Result};
use rustral_nn::{Batch, CacheConfig, CacheQuantization};

use crate::device::{Ctx, DeviceBuffer};
use crate::error::check;
use crate::ffi;
use crate::tensor::{DType, RocmTensor};
use crate::RocmBackend;

/// Storage of the pools.
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum KvDtype {
    F32,
    Bf16,
    Int8,
    Fp8,
}

impl KvDtype {
    fn code(self) -> i32 {
        match self {
            KvDtype::F32 => ffi::RKV_F32,
            KvDtype::Bf16 => ffi::RKV_BF16,
            KvDtype::Int8 => ffi::RKV_I8,
            KvDtype::Fp8 => ffi::RKV_FP8,
        }
    }
    fn size(self) -> usize {
        match self {
            KvDtype::F32 => 4,
            KvDtype::Bf16 => 2,
            KvDtype::Int8 | KvDtype::Fp8 => 1,
        }
    }
    fn one_byte(self) -> bool {
        matches!(self, KvDtype::Int8 | KvDtype::Fp8)
    }
    /// The reference's cache quantization (crates/nn/src/kv_cache.rs:38-63):
    /// Fp16 is stored as bf16 (round to nearest even), Fp8 as OCP e4m3 with a
    /// per-row scale, Int8 as int8 with a per-row scale.
    pub fn from_quantization(q: CacheQuantization) -> Self {
        match q {
            CacheQuantization::Fp32 => KvDtype::F32,
            CacheQuantization::Fp16 => KvDtype::Bf16,
            CacheQuantization::Fp8 => KvDtype::Fp8,
            CacheQuantization::Int8 => KvDtype::Int8,
        }
    }
}

#[derive(Clone, Debug)]
pub struct PagedKvConfig {
    pub layers: usize,
    pub num_blocks: usize,
    pub num_kv_heads: usize,
    pub head_dim: usize,
    pub dtype: KvDtype,
}

pub const BLOCK_SIZE: usize = 16;

pub struct RocmPagedKvCache {
    ctx: Arc<Ctx>,
    cfg: PagedKvConfig,
    k: DeviceBuffer,
    v: DeviceBuffer,
    k_scale: Option<DeviceBuffer>,
    v_scale: Option<DeviceBuffer>,
    /// split-K partials of decode attention, grown on demand
    ws: Mutex<DeviceBuffer>,
}

fn ci(v: usize, what: &str) -> Result<i32> {
    i32::try_from(v).map_err(|_| CoreError::InvalidArgument(format!("{what} = {v} exceeds i32")))
}

/// The shapes an attention call's kernels index by: q rows `[n, Hq, D]`
/// with `D` the pool's head_dim and `Hq` a multiple of its KV heads, and one
/// table row and one length per sequence (`seqs` of them; `q_start` when
/// given holds `seqs + 1` offsets).  The kernels take sizes, not buffer
/// lengths, so a mismatch here would read past the tables or write rows of
/// the wrong width into the pools: it is rejected before any launch.
pub(crate) fn check_attention_shapes(cfg: &PagedKvConfig, q: &[usize], block_tables: &[usize], ctx_lens: &[usize],
                                     q_start: Option<&[usize]>) -> Result<()> {
    let bad = |m: String| Err(CoreError::InvalidArgument(m));
    if q.len() != 3 || block_tables.len() != 2 || ctx_lens.len() != 1 {
        let ranks = (q.len(), block_tables.len(), ctx_lens.len());
        return bad(format!("attention: q, block_tables and ctx_lens have ranks {ranks:?}, not (3, 2, 1)"));
    }
    if q[2] != cfg.head_dim {
        return bad(format!("attention: q head_dim {} differs from the pool's {}", q[2], cfg.head_dim));
    }
    if q[1] == 0 || q[1] % cfg.num_kv_heads != 0 {
        return bad(format!("attention: {} query heads are not a multiple of {} KV heads", q[1], cfg.num_kv_heads));
    }
    let seqs = ctx_lens[0];
    if block_tables[0] != seqs {
        return bad(format!("attention: {} block-table rows for {seqs} sequences", block_tables[0]));
    }
    match q_start {
        Some(qs) if qs.len() != 1 || qs[0] != seqs + 1 => {
            bad(format!("attention: q_start {qs:?} must hold {} offsets", seqs + 1))
        }
        None if q[0] != seqs => bad(format!("attention: {} q rows for {seqs} sequences", q[0])),
        _ => Ok(()),
    }
}

impl RocmPagedKvCache {
    pub fn new(backend: &RocmBackend, cfg: PagedKvConfig) -> Result<Self> {
        let ctx = backend.ctx.clone();
        let rows = cfg.layers * cfg.num_blocks * cfg.num_kv_heads * BLOCK_SIZE;
        let bytes = rows * cfg.head_dim * cfg.dtype.size();
        let k = DeviceBuffer::zeroed(&ctx, bytes)?;
        let v = DeviceBuffer::zeroed(&ctx, bytes)?;
        let (k_scale, v_scale) = if cfg.dtype.one_byte() {
            (Some(DeviceBuffer::zeroed(&ctx, rows * 4)?), Some(DeviceBuffer::zeroed(&ctx, rows * 4)?))
        } else {
            (None, None)
        };
        let ws = Mutex::new(DeviceBuffer::new(0)?);
        Ok(Self { ctx, cfg, k, v, k_scale, v_scale, ws })
    }

    /// Pools for the reference's `CacheConfig` (crates/nn/src/kv_cache.rs:
    /// 115-134): its KV heads, head_dim and quantization, `layers` layers of
    /// `num_blocks` 16-token blocks.
    pub fn from_cache_config(backend: &RocmBackend, c: &CacheConfig, layers: usize, num_blocks: usize) -> Result<Self> {
        Self::new(backend, PagedKvConfig {
            layers,
            num_blocks,
            num_kv_heads: c.num_kv_heads,
            head_dim: c.head_dim,
            dtype: KvDtype::from_quantization(c.quantization),
        })
    }

    pub fn config(&self) -> &PagedKvConfig {
        &self.cfg
    }

    fn layer_elems(&self) -> usize {
        self.cfg.num_blocks * self.cfg.num_kv_heads * BLOCK_SIZE * self.cfg.head_dim
    }

    fn layer_ptr(&self, buf: &DeviceBuffer, layer: usize) -> Result<*mut c_void> {
        if layer >= self.cfg.layers {
            return Err(CoreError::InvalidArgument(format!("layer {layer} of {}", self.cfg.layers)));
        }
        // SAFETY: the offset lies inside the all-layer allocation.
        Ok(unsafe { (buf.ptr() as *mut u8).add(layer * self.layer_elems() * self.cfg.dtype.size()) } as *mut c_void)
    }

    fn scale_ptr(&self, buf: &Option<DeviceBuffer>, layer: usize) -> *mut f32 {
        match buf {
            // SAFETY: the offset lies inside the all-layer scale allocation.
            Some(b) => unsafe {
                (b.ptr() as *mut f32).add(layer * self.cfg.num_blocks * self.cfg.num_kv_heads * BLOCK_SIZE)
            },
            None => std::ptr::null_mut(),
        }
    }

    /// Replaces `KVCache::append` (crates/nn/src/kv_cache.rs:172-216): new K
    /// and V rows `[layers, n_tokens, Hkv, D]` (every layer in one launch) or
    /// `[n_tokens, Hkv, D]` (layer 0) go to the int64 pool slots of
    /// `slot_mapping` (`block * 16 + row`; negative: skipped).
    pub fn append(&mut self, k_new: &RocmTensor, v_new: &RocmTensor, slot_mapping: &RocmTensor) -> Result<()> {
        slot_mapping.expect(DType::I64, 1, "slot_mapping")?;
        let (layers, n_tok) = match k_new.shape.as_slice() {
            [l, n, h, d] if *h == self.cfg.num_kv_heads && *d == self.cfg.head_dim => (*l, *n),
            [n, h, d] if *h == self.cfg.num_kv_heads && *d == self.cfg.head_dim => (1, *n),
            _ => return Err(CoreError::InvalidArgument(format!("k_new shape {:?}", k_new.shape))),
        };
        if v_new.shape != k_new.shape || layers > self.cfg.layers || slot_mapping.shape[0] != n_tok {
            return Err(CoreError::InvalidArgument("append: K / V / slot shapes disagree".into()));
        }
        let (h, d) = (self.cfg.num_kv_heads, self.cfg.head_dim);
        let tok = (h * d) as i64;
        let le = self.layer_elems() as i64;
        let s = self.ctx.stream;
        let code = self.cfg.dtype.code();
        // SAFETY: pools, scales, sources and slots are live device buffers of the shapes checked above.
        let rc = unsafe {
            if self.cfg.dtype.one_byte() {
                ffi::rkv_append_q(self.k.ptr(), self.v.ptr(), self.scale_ptr(&self.k_scale, 0),
                                  self.scale_ptr(&self.v_scale, 0), le, k_new.device_ptr() as *const f32,
                                  v_new.device_ptr() as *const f32, n_tok as i64 * tok, tok, d as i64,
                                  slot_mapping.device_ptr() as *const i64, n_tok as i64, ci(layers, "layers")?,
                                  ci(h, "heads")?, ci(d, "head_dim")?, BLOCK_SIZE as i32,
                                  self.cfg.num_blocks as i64, code, s)
            } else {
                ffi::rkv_append(self.k.ptr(), self.v.ptr(), le, k_new.device_ptr() as *const f32,
                                v_new.device_ptr() as *const f32, n_tok as i64 * tok, tok, d as i64,
                                slot_mapping.device_ptr() as *const i64, n_tok as i64, ci(layers, "layers")?,
                                ci(h, "heads")?, ci(d, "head_dim")?, BLOCK_SIZE as i32,
                                self.cfg.num_blocks as i64, code, s)
            }
        };
        check(rc)
    }

    /// Replaces `KVCache::get_range` / `k_cache` / `v_cache`
    /// (crates/nn/src/kv_cache.rs:219-243): each sequence's K and V in the
    /// reference's `[B, Hkv, max_ctx, D]` layout (fp32 for fp32 and 1-byte
    /// pools, bf16 bits for bf16 pools); rows past a sequence's length are
    /// left unwritten.
    pub fn gather(&self, layer: usize, block_tables: &RocmTensor, ctx_lens: &RocmTensor, max_ctx: usize)
        -> Result<(RocmTensor, RocmTensor)> {
        block_tables.expect(DType::I32, 2, "block_tables")?;
        ctx_lens.expect(DType::I32, 1, "ctx_lens")?;
        if ctx_lens.shape[0] != block_tables.shape[0] {
            return Err(CoreError::InvalidArgument(format!(
                "gather: {} block-table rows for {} lengths", block_tables.shape[0], ctx_lens.shape[0]
            )));
        }
        let (b, mb) = (block_tables.shape[0], block_tables.shape[1]);
        let (h, d) = (self.cfg.num_kv_heads, self.cfg.head_dim);
        let out_dt = if self.cfg.dtype == KvDtype::Bf16 { DType::Bf16 } else { DType::F32 };
        let shape = [b, h, max_ctx, d];
        let ko = RocmTensor::empty(&self.ctx, &shape, out_dt)?;
        let vo = RocmTensor::empty(&self.ctx, &shape, out_dt)?;
        let (kp, vp) = (self.layer_ptr(&self.k, layer)?, self.layer_ptr(&self.v, layer)?);
        // SAFETY: live buffers: one table row per length, outputs allocated here
        // at [b, h, max_ctx, d] (the kernel clamps each length to max_ctx).
        let rc = unsafe {
            if self.cfg.dtype.one_byte() {
                ffi::rkv_gather_q(ko.device_ptr() as *mut f32, vo.device_ptr() as *mut f32, kp, vp,
                                  self.scale_ptr(&self.k_scale, layer), self.scale_ptr(&self.v_scale, layer),
                                  block_tables.device_ptr() as *const i32, ci(mb, "max_blocks")?,
                                  ctx_lens.device_ptr() as *const i32, std::ptr::null(), ci(b, "B")?, ci(h, "heads")?,
                                  ci(d, "head_dim")?, BLOCK_SIZE as i32, self.cfg.num_blocks as i64,
                                  ci(max_ctx, "max_ctx")?, self.cfg.dtype.code(), self.ctx.stream)
            } else {
                ffi::rkv_gather(ko.device_ptr(), vo.device_ptr(), kp, vp, block_tables.device_ptr() as *const i32,
                                ci(mb, "max_blocks")?, ctx_lens.device_ptr() as *const i32, std::ptr::null(),
                                ci(b, "B")?, ci(h, "heads")?, ci(d, "head_dim")?, BLOCK_SIZE as i32,
                                self.cfg.num_blocks as i64, ci(max_ctx, "max_ctx")?, self.cfg.dtype.code(),
                                self.cfg.dtype.code(), self.ctx.stream)
            }
        };
        check(rc)?;
        Ok((ko, vo))
    }

    /// Compaction for continuous batching (no reference counterpart:
    /// `PagedCache` only frees, crates/nn/src/continuous_batching.rs:380-386):
    /// block `pairs[i][1] := pairs[i][0]` in every layer, K, V and scales.
    /// Sources and destinations must be disjoint.
    pub fn copy_blocks(&mut self, pairs: &RocmTensor) -> Result<()> {
        pairs.expect(DType::I32, 2, "pairs")?;
        if pairs.shape[1] != 2 {
            return Err(CoreError::InvalidArgument(format!("copy_blocks: pairs {:?} must be [n, 2]", pairs.shape)));
        }
        let n = ci(pairs.shape[0], "pairs")?;
        let block_bytes = (self.cfg.num_kv_heads * BLOCK_SIZE * self.cfg.head_dim * self.cfg.dtype.size()) as i64;
        let ls = self.layer_elems() as i64 * self.cfg.dtype.size() as i64;
        let (layers, s) = (ci(self.cfg.layers, "layers")?, self.ctx.stream);
        // SAFETY: pools and pairs are live device buffers.
        check(unsafe {
            ffi::rkv_copy_blocks(self.k.ptr(), self.v.ptr(), ls, layers, pairs.device_ptr() as *const i32, n,
                                 block_bytes, self.cfg.num_blocks as i64, s)
        })?;
        if let (Some(ks), Some(vs)) = (&self.k_scale, &self.v_scale) {
            let sb = (self.cfg.num_kv_heads * BLOCK_SIZE * 4) as i64;
            // SAFETY: as above, on the scale pools.
            check(unsafe {
                ffi::rkv_copy_blocks(ks.ptr(), vs.ptr(), sb * self.cfg.num_blocks as i64, layers,
                                     pairs.device_ptr() as *const i32, n, sb, self.cfg.num_blocks as i64, s)
            })?;
        }
        Ok(())
    }

    /// One decode token of every sequence (the per-head recipe of
    /// `TapeMultiHeadAttention::forward_tape_with_mask`,
    /// crates/nn/src/tape_transformer.rs:87-139, with GQA): q `[B, Hq, D]`
    /// fp32 -> out `[B, Hq, D]`, `softmax((q . K) * scale) V` over each
    /// sequence's `ctx_lens[b]` cached tokens.
    pub fn decode_attention(&self, layer: usize, q: &RocmTensor, block_tables: &RocmTensor, ctx_lens: &RocmTensor,
                            max_context: usize, scale: f32) -> Result<RocmTensor> {
        q.expect(DType::F32, 3, "q")?;
        block_tables.expect(DType::I32, 2, "block_tables")?;
        ctx_lens.expect(DType::I32, 1, "ctx_lens")?;
        check_attention_shapes(&self.cfg, &q.shape, &block_tables.shape, &ctx_lens.shape, None)?;
        let (b, hq, d) = (q.shape[0], q.shape[1], q.shape[2]);
        let mb = block_tables.shape[1];
        let need = unsafe {
            // SAFETY: pure size computation in the library.
            ffi::rkv_decode_workspace_bytes(ci(b, "B")?, ci(hq, "Hq")?, ci(d, "D")?, ci(max_context, "max_context")?, 0)
        };
        let mut ws = self.ws.lock().map_err(|_| CoreError::Backend("workspace lock poisoned".into()))?;
        if ws.bytes() < need {
            // the stream may still read the old partials: drain it first
            self.ctx.synchronize()?;
            *ws = DeviceBuffer::new(need)?;
        }
        let out = RocmTensor::empty(&self.ctx, &q.shape, DType::F32)?;
        let (kp, vp) = (self.layer_ptr(&self.k, layer)?, self.layer_ptr(&self.v, layer)?);
        // SAFETY: live buffers whose shapes check_attention_shapes has matched to
        // the pool; the workspace holds `need` bytes.
        let rc = unsafe {
            if self.cfg.dtype.one_byte() {
                ffi::rkv_decode_attention_q(out.device_ptr() as *mut f32, q.device_ptr() as *const f32, kp, vp,
                                            self.scale_ptr(&self.k_scale, layer), self.scale_ptr(&self.v_scale, layer),
                                            block_tables.device_ptr() as *const i32, ci(mb, "max_blocks")?,
                                            ctx_lens.device_ptr() as *const i32, ci(b, "B")?, ci(hq, "Hq")?,
                                            ci(self.cfg.num_kv_heads, "Hkv")?, ci(d, "D")?, BLOCK_SIZE as i32,
                                            self.cfg.num_blocks as i64, ci(max_context, "max_context")?, scale,
                                            self.cfg.dtype.code(), 0, ws.ptr(), ws.bytes(), self.ctx.stream)
            } else {
                ffi::rkv_decode_attention(out.device_ptr() as *mut f32, q.device_ptr() as *const f32, kp, vp,
                                          block_tables.device_ptr() as *const i32, ci(mb, "max_blocks")?,
                                          ctx_lens.device_ptr() as *const i32, ci(b, "B")?, ci(hq, "Hq")?,
                                          ci(self.cfg.num_kv_heads, "Hkv")?, ci(d, "D")?, BLOCK_SIZE as i32,
                                          self.cfg.num_blocks as i64, ci(max_context, "max_context")?, scale,
                                          self.cfg.dtype.code(), 0, ws.ptr(), ws.bytes(), self.ctx.stream)
            }
        };
        check(rc)?;
        Ok(out)
    }

    /// One decode step of layer `layer` with its K/V append fused in:
    /// `ctx_lens` already counts the new token, whose rows `k_new` / `v_new`
    /// `[B, Hkv, D]` f32 go to position `ctx_lens[b] - 1` (bf16 pools
    /// rounded, 1-byte pools quantized with their row scale).  Equals
    /// `append` of those rows followed by `decode_attention`, in one launch
    /// (`KVCache::append`, crates/nn/src/kv_cache.rs:172-216, then the
    /// attention of crates/nn/src/tape_transformer.rs:87-139).
    pub fn decode_attention_append(&self, layer: usize, q: &RocmTensor, k_new: &RocmTensor, v_new: &RocmTensor,
                                   block_tables: &RocmTensor, ctx_lens: &RocmTensor, max_context: usize,
                                   scale: f32) -> Result<RocmTensor> {
        if self.cfg.dtype == KvDtype::F32 {
            return Err(CoreError::InvalidArgument("the fused append + decode needs a bf16 or 1-byte pool".into()));
        }
        q.expect(DType::F32, 3, "q")?;
        k_new.expect(DType::F32, 3, "k_new")?;
        v_new.expect(DType::F32, 3, "v_new")?;
        block_tables.expect(DType::I32, 2, "block_tables")?;
        ctx_lens.expect(DType::I32, 1, "ctx_lens")?;
        check_attention_shapes(&self.cfg, &q.shape, &block_tables.shape, &ctx_lens.shape, None)?;
        let (b, hq, d) = (q.shape[0], q.shape[1], q.shape[2]);
        let rows = [b, self.cfg.num_kv_heads, d];
        for t in [k_new, v_new] {
            if t.shape[..] != rows[..] {
                return Err(CoreError::ShapeMismatch { expected: rows.to_vec(), actual: t.shape.clone() });
            }
        }
        let mb = block_tables.shape[1];
        let need = unsafe {
            // SAFETY: pure size computation in the library.
            ffi::rkv_decode_workspace_bytes(ci(b, "B")?, ci(hq, "Hq")?, ci(d, "D")?, ci(max_context, "max_context")?, 0)
        };
        let mut ws = self.ws.lock().map_err(|_| CoreError::Backend("workspace lock poisoned".into()))?;
        if ws.bytes() < need {
            self.ctx.synchronize()?;
            *ws = DeviceBuffer::new(need)?;
        }
        let out = RocmTensor::empty(&self.ctx, &q.shape, DType::F32)?;
        let (kp, vp) = (self.layer_ptr(&self.k, layer)?, self.layer_ptr(&self.v, layer)?);
        // SAFETY: live buffers whose shapes check_attention_shapes and the row
        // check above have matched to the pool; the workspace holds `need` bytes.
        let rc = unsafe {
            if self.cfg.dtype.one_byte() {
                ffi::rkv_decode_attention_append_q(out.device_ptr() as *mut f32, q.device_ptr() as *const f32, kp, vp,
                                                   self.scale_ptr(&self.k_scale, layer),
                                                   self.scale_ptr(&self.v_scale, layer),
                                                   k_new.device_ptr() as *const f32, v_new.device_ptr() as *const f32,
                                                   block_tables.device_ptr() as *const i32, ci(mb, "max_blocks")?,
                                                   ctx_lens.device_ptr() as *const i32, ci(b, "B")?, ci(hq, "Hq")?,
                                                   ci(self.cfg.num_kv_heads, "Hkv")?, ci(d, "D")?, BLOCK_SIZE as i32,
                                                   self.cfg.num_blocks as i64, ci(max_context, "max_context")?, scale,
                                                   self.cfg.dtype.code(), 0, ws.ptr(), ws.bytes(), self.ctx.stream)
            } else {
                ffi::rkv_decode_attention_append(out.device_ptr() as *mut f32, q.device_ptr() as *const f32, kp, vp,
                                                 k_new.device_ptr() as *const f32, v_new.device_ptr() as *const f32,
                                                 block_tables.device_ptr() as *const i32, ci(mb, "max_blocks")?,
                                                 ctx_lens.device_ptr() as *const i32, ci(b, "B")?, ci(hq, "Hq")?,
                                                 ci(self.cfg.num_kv_heads, "Hkv")?, ci(d, "D")?, BLOCK_SIZE as i32,
                                                 self.cfg.num_blocks as i64, ci(max_context, "max_context")?, scale,
                                                 ffi::RKV_BF16, 0, ws.ptr(), ws.bytes(), self.ctx.stream)
            }
        };
        check(rc)?;
        Ok(out)
    }

    /// Causal prefill of new tokens already appended: sequence b's query rows
    /// `q_start[b]..q_start[b+1]` are its last tokens and attend to every
    /// cached position up to their own (`forward_tape_with_mask` with
    /// `causal_mask_tape`, crates/nn/src/tape_transformer.rs:87-139, :276-296).
    #[allow(clippy::too_many_arguments)]
    pub fn prefill_attention(&self, layer: usize, q: &RocmTensor, block_tables: &RocmTensor, q_start: &RocmTensor,
                             ctx_lens: &RocmTensor, max_q_len: usize, scale: f32) -> Result<RocmTensor> {
        q.expect(DType::F32, 3, "q")?;
        block_tables.expect(DType::I32, 2, "block_tables")?;
        q_start.expect(DType::I32, 1, "q_start")?;
        ctx_lens.expect(DType::I32, 1, "ctx_lens")?;
        check_attention_shapes(&self.cfg, &q.shape, &block_tables.shape, &ctx_lens.shape, Some(&q_start.shape))?;
        if self.cfg.dtype.one_byte() {
            return Err(CoreError::Backend("prefill_attention: 1-byte pools are not built".into()));
        }
        let b = ctx_lens.shape[0];
        let out = RocmTensor::empty(&self.ctx, &q.shape, DType::F32)?;
        let (kp, vp) = (self.layer_ptr(&self.k, layer)?, self.layer_ptr(&self.v, layer)?);
        // SAFETY: live buffers whose shapes check_attention_shapes has matched to
        // the pool; q_start's values are device data the caller vouches for
        // (rows q_start[b]..q_start[b + 1] lie inside q, rkv_prefill_attention's
        // contract).
        check(unsafe {
            ffi::rkv_prefill_attention(out.device_ptr() as *mut f32, q.device_ptr() as *const f32, kp, vp,
                                       block_tables.device_ptr() as *const i32, ci(block_tables.shape[1], "max_blocks")?,
                                       q_start.device_ptr() as *const i32, ctx_lens.device_ptr() as *const i32,
                                       ci(b, "B")?, ci(q.shape[1], "Hq")?, ci(self.cfg.num_kv_heads, "Hkv")?,
                                       ci(q.shape[2], "D")?, BLOCK_SIZE as i32, self.cfg.num_blocks as i64,
                                       ci(max_q_len, "max_q_len")?, scale, self.cfg.dtype.code(), self.ctx.stream)
        })?;
        Ok(out)
    }
}

/// The scheduler's `Batch` (crates/nn/src/continuous_batching.rs:157-167) as
/// the device arrays the paged calls take: block tables `[B, max_blocks]`
/// int32 (-1 padded) and sequence lengths `[B]` int32, one upload each.
pub fn batch_to_device(backend: &RocmBackend, batch: &Batch) -> Result<(RocmTensor, RocmTensor)> {
    let b = batch.block_tables.len();
    let mb = batch.block_tables.iter().map(|t| t.len()).max().unwrap_or(0).max(1);
    let mut tab = vec![-1i32; b * mb];
    for (i, t) in batch.block_tables.iter().enumerate() {
        for (j, &blk) in t.iter().enumerate() {
            tab[i * mb + j] = ci(blk, "block id")?;
        }
    }
    let lens: Vec<i32> = batch.seq_lens.iter().map(|&l| ci(l, "seq_len")).collect::<Result<_>>()?;
    Ok((
        RocmTensor::upload(&backend.ctx, &tab, &[b, mb], DType::I32)?,
        RocmTensor::upload(&backend.ctx, &lens, &[lens.len()], DType::I32)?,
    ))
}

#[cfg(test)]
mod tests {
    use super::*;

    fn cfg() -> PagedKvConfig {
        PagedKvConfig { layers: 2, num_blocks: 64, num_kv_heads: 8, head_dim: 128, dtype: KvDtype::Bf16 }
    }

    #[test]
    fn matching_decode_and_prefill_shapes_pass() {
        let c = cfg();
        assert!(check_attention_shapes(&c, &[4, 32, 128], &[4, 16], &[4], None).is_ok());
        assert!(check_attention_shapes(&c, &[300, 32, 128], &[4, 16], &[4], Some(&[5])).is_ok());
    }

    #[test]
    fn mismatched_shapes_are_rejected_before_a_launch() {
        let c = cfg();
        let err = |r: Result<()>| matches!(r, Err(CoreError::InvalidArgument(_)));
        // a head_dim other than the pool's: rows of the wrong width into the pool
        assert!(err(check_attention_shapes(&c, &[4, 32, 256], &[4, 16], &[4], None)));
        assert!(err(check_attention_shapes(&c, &[4, 32, 64], &[4, 16], &[4], None)));
        // query heads not a multiple of the KV heads
        assert!(err(check_attention_shapes(&c, &[4, 12, 128], &[4, 16], &[4], None)));
        assert!(err(check_attention_shapes(&c, &[4, 0, 128], &[4, 16], &[4], None)));
        // short tables or lengths: the kernel would read past them
        assert!(err(check_attention_shapes(&c, &[4, 32, 128], &[3, 16], &[4], None)));
        assert!(err(check_attention_shapes(&c, &[4, 32, 128], &[4, 16], &[3], None)));
        assert!(err(check_attention_shapes(&c, &[5, 32, 128], &[4, 16], &[4], None)));
        // prefill offsets: B + 1 of them
        assert!(err(check_attention_shapes(&c, &[300, 32, 128], &[4, 16], &[4], Some(&[4]))));
        // ranks
        assert!(err(check_attention_shapes(&c, &[4, 32], &[4, 16], &[4], None)));
    }
}
