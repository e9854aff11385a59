//! The callers either side of the paged calls: the block manager in its
//! host form (`rkv_bm_*`, `PagedCache` semantics with tables that grow by
//! append) and its device-resident form (`rkv_dbm_*`, state in HBM, calls
//! enqueued on the backend's stream and capturable in a HIP graph).

use std::sync::Arc;

use rustral_core::{CoreError, Result};

use crate::device::Ctx;
use crate::error::{check, last_error};
use crate::ffi;
use crate::tensor::{DType, RocmTensor};
use crate::RocmBackend;

/// `PagedCache` (crates/nn/src/kv_cache.rs:381-432): FIFO free list of block
/// ids; `allocate` takes `ceil(tokens / block_size)` ids (None when the pool
/// is short), `free` gives a sequence's ids back.  A sequence's table is
/// appended to (the reference overwrites it, :422).
pub struct BlockManager {
    h: *mut ffi::RkvBlockManager,
}

// SAFETY: the handle is used through &mut self only (or read through &self).
unsafe impl Send for BlockManager {}

impl BlockManager {
    pub fn new(num_blocks: usize, block_size: usize) -> Result<Self> {
        // SAFETY: plain constructor call.
        let h = unsafe { ffi::rkv_bm_create(num_blocks as i64, block_size as i32) };
        if h.is_null() {
            return Err(CoreError::Backend(last_error()));
        }
        Ok(Self { h })
    }

    /// The ids taken, or None on OOM (the reference's `None`, :416-418).
    pub fn allocate(&mut self, seq: u64, num_tokens: usize) -> Option<Vec<usize>> {
        let want = (num_tokens + self.block_size() - 1) / self.block_size();
        let mut ids = vec![0i32; want.max(1)];
        // SAFETY: ids holds `want` entries.
        let n = unsafe { ffi::rkv_bm_allocate(self.h, seq as i64, num_tokens as i64, ids.as_mut_ptr(), want as i64) };
        if n < 0 {
            return None;
        }
        Some(ids[..n as usize].iter().map(|&b| b as usize).collect())
    }

    pub fn free(&mut self, seq: u64) -> usize {
        // SAFETY: valid handle.
        unsafe { ffi::rkv_bm_free(self.h, seq as i64).max(0) as usize }
    }

    pub fn num_free(&self) -> usize {
        // SAFETY: valid handle.
        unsafe { ffi::rkv_bm_num_free(self.h).max(0) as usize }
    }

    pub fn block_size(&self) -> usize {
        // SAFETY: valid handle.
        unsafe { ffi::rkv_bm_block_size(self.h).max(1) as usize }
    }

    pub fn table(&self, seq: u64) -> Vec<usize> {
        // SAFETY: a NULL buffer asks for the length only; then a buffer of that length.
        unsafe {
            let n = ffi::rkv_bm_table(self.h, seq as i64, std::ptr::null_mut(), 0);
            if n <= 0 {
                return Vec::new();
            }
            let mut v = vec![0i32; n as usize];
            ffi::rkv_bm_table(self.h, seq as i64, v.as_mut_ptr(), n);
            v.into_iter().map(|b| b as usize).collect()
        }
    }

    /// Compaction plan: up to `max_moves` (src, dst) pairs moving live blocks
    /// into lower free ids; the tables are updated, `copy_blocks` moves the
    /// bytes.
    pub fn plan_compaction(&mut self, max_moves: usize) -> Vec<(usize, usize)> {
        let mut pairs = vec![0i32; 2 * max_moves.max(1)];
        // SAFETY: pairs holds 2 * max_moves entries.
        let n = unsafe { ffi::rkv_bm_plan_compaction(self.h, max_moves as i64, pairs.as_mut_ptr(), max_moves as i64) };
        (0..n.max(0) as usize).map(|i| (pairs[2 * i] as usize, pairs[2 * i + 1] as usize)).collect()
    }
}

impl BlockManager {
    /// Migration plan: `min(max_moves, live, free)` live blocks move, highest
    /// id first, to the lowest free ids (no stop above the source).
    pub fn plan_migration(&mut self, max_moves: usize) -> Vec<(usize, usize)> {
        let mut pairs = vec![0i32; 2 * max_moves.max(1)];
        // SAFETY: pairs holds 2 * max_moves entries.
        let n = unsafe { ffi::rkv_bm_plan_migration(self.h, max_moves as i64, pairs.as_mut_ptr(), max_moves as i64) };
        (0..n.max(0) as usize).map(|i| (pairs[2 * i] as usize, pairs[2 * i + 1] as usize)).collect()
    }
}

impl BlockManager {
    /// Relocation plan: the blocks `plan_migration` would move, into the
    /// longest runs of free ids (longest first), pairs ascending on both
    /// sides so `copy_blocks` writes runs of consecutive blocks.
    pub fn plan_relocation(&mut self, max_moves: usize) -> Vec<(usize, usize)> {
        let mut pairs = vec![0i32; 2 * max_moves.max(1)];
        // SAFETY: pairs holds 2 * max_moves entries.
        let n = unsafe { ffi::rkv_bm_plan_relocation(self.h, max_moves as i64, pairs.as_mut_ptr(), max_moves as i64) };
        (0..n.max(0) as usize).map(|i| (pairs[2 * i] as usize, pairs[2 * i + 1] as usize)).collect()
    }
}

impl Drop for BlockManager {
    fn drop(&mut self) {
        // SAFETY: created by rkv_bm_create, destroyed once.
        unsafe { ffi::rkv_bm_destroy(self.h) }
    }
}

/// The block manager with its state in device memory: per step
/// `reserve(slots, lengths)` grows the tables, `slot_mapping` gives `append`
/// its int64 slots and `batch_tables` gives the attention calls their
/// tables, all stream-ordered; `status` is the one synchronising call.
pub struct DeviceBlockManager {
    h: *mut ffi::RkvDeviceBlockManager,
    ctx: Arc<Ctx>,
    max_blocks_per_seq: usize,
}

// SAFETY: calls are ordered on the backend's stream; the handle is only read.
unsafe impl Send for DeviceBlockManager {}
unsafe impl Sync for DeviceBlockManager {}

impl DeviceBlockManager {
    pub fn new(backend: &RocmBackend, num_blocks: usize, max_seqs: usize, max_blocks_per_seq: usize) -> Result<Self> {
        // SAFETY: plain constructor call on the backend's stream.
        let h = unsafe {
            ffi::rkv_dbm_create(num_blocks as i64, 16, max_seqs as i32, max_blocks_per_seq as i32, backend.ctx.stream)
        };
        if h.is_null() {
            return Err(CoreError::Backend(last_error()));
        }
        Ok(Self { h, ctx: backend.ctx.clone(), max_blocks_per_seq })
    }

    /// Grows every listed slot's table to cover `num_tokens[i]` tokens
    /// (all-or-nothing; a failure is reported by `status`).
    pub fn reserve(&self, slots: &RocmTensor, num_tokens: &RocmTensor) -> Result<()> {
        slots.expect(DType::I32, 1, "slots")?;
        num_tokens.expect(DType::I32, 1, "num_tokens")?;
        // SAFETY: device int32 arrays of slots.numel() entries.
        check(unsafe {
            ffi::rkv_dbm_reserve(self.h, slots.device_ptr() as *const i32, num_tokens.device_ptr() as *const i32,
                                 slots.numel() as i32, self.ctx.stream)
        })
    }

    pub fn free(&self, slots: &RocmTensor) -> Result<()> {
        slots.expect(DType::I32, 1, "slots")?;
        // SAFETY: as above.
        check(unsafe { ffi::rkv_dbm_free(self.h, slots.device_ptr() as *const i32, slots.numel() as i32, self.ctx.stream) })
    }

    /// Pool slots (`block * 16 + row`) of (slot, position) pairs, int64.
    pub fn slot_mapping(&self, slots: &RocmTensor, positions: &RocmTensor) -> Result<RocmTensor> {
        slots.expect(DType::I32, 1, "slots")?;
        positions.expect(DType::I32, 1, "positions")?;
        let out = RocmTensor::empty(&self.ctx, &[slots.numel()], DType::I64)?;
        // SAFETY: device arrays of n entries.
        check(unsafe {
            ffi::rkv_dbm_slot_mapping(self.h, slots.device_ptr() as *const i32, positions.device_ptr() as *const i32,
                                      slots.numel() as i32, out.device_ptr() as *mut i64, self.ctx.stream)
        })?;
        Ok(out)
    }

    /// Dense `[n, max_blocks_per_seq]` tables of the listed slots.
    pub fn batch_tables(&self, slots: &RocmTensor) -> Result<RocmTensor> {
        slots.expect(DType::I32, 1, "slots")?;
        let out = RocmTensor::empty(&self.ctx, &[slots.numel(), self.max_blocks_per_seq], DType::I32)?;
        // SAFETY: out holds n * max_blocks entries.
        check(unsafe {
            ffi::rkv_dbm_batch_tables(self.h, slots.device_ptr() as *const i32, slots.numel() as i32,
                                      out.device_ptr() as *mut i32, self.max_blocks_per_seq as i32, self.ctx.stream)
        })?;
        Ok(out)
    }

    /// (free blocks, error flags) after everything enqueued so far; a set
    /// `RKV_DBM_ERR_OOM` flag is the host manager's OOM.
    pub fn status(&self, clear: bool) -> Result<(i64, i32)> {
        let (mut nf, mut err) = (0i64, 0i32);
        // SAFETY: host out-pointers.
        check(unsafe { ffi::rkv_dbm_status(self.h, &mut nf, &mut err, clear as i32, self.ctx.stream) })?;
        Ok((nf, err))
    }
}

impl Drop for DeviceBlockManager {
    fn drop(&mut self) {
        // SAFETY: created by rkv_dbm_create, destroyed once.
        unsafe { ffi::rkv_dbm_destroy(self.h) }
    }
}
