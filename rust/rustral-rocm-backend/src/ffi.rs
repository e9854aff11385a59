//! Raw declarations of the C ABI of librustral_kv: every function of
//! include/rustral_kv.h, include/rustral_serving.h and include/rustral_model.h,
//! in header order, with the C types mapped one to one (`int` -> `c_int`,
//! `int32_t` -> `i32`, `int64_t` -> `i64`, `size_t` -> `usize`, pointers to
//! `*const` / `*mut` of the same element type; `void* stream` is a
//! `hipStream_t`).  A CPU test of the repository parses this file and the
//! headers and checks names, arity and every parameter's width.
#![allow(non_camel_case_types, dead_code)]

use std::os::raw::{c_char, c_int, c_void};

/// `hipStream_t` (NULL: the device's null stream).
pub type Stream = *mut c_void;

pub const RKV_F32: c_int = 0;
pub const RKV_BF16: c_int = 1;
pub const RKV_I8: c_int = 2;
pub const RKV_FP8: c_int = 3;

pub const RKV_OK: c_int = 0;
pub const RKV_ERR_INVALID_ARG: c_int = -1;
pub const RKV_ERR_UNSUPPORTED: c_int = -2;
pub const RKV_ERR_WORKSPACE: c_int = -3;
pub const RKV_ERR_HIP: c_int = -4;
pub const RKV_ERR_OOM: c_int = -5;

pub const RKV_DBM_ERR_OOM: i32 = 1;
pub const RKV_DBM_ERR_TABLE_FULL: i32 = 2;
pub const RKV_DBM_ERR_ARG: i32 = 4;

pub const RKV_PRIORITY_LOW: c_int = 0;
pub const RKV_PRIORITY_NORMAL: c_int = 1;
pub const RKV_PRIORITY_HIGH: c_int = 2;
pub const RKV_PRIORITY_CRITICAL: c_int = 3;
pub const RKV_EOS_TOKEN: i32 = 2;

/// `rkv_decoder_config` (include/rustral_model.h).
#[repr(C)]
#[derive(Clone, Copy, Debug, PartialEq)]
pub struct RkvDecoderConfig {
    pub vocab: c_int,
    pub d_model: c_int,
    pub n_heads: c_int,
    pub n_kv_heads: c_int,
    pub d_ff: c_int,
    pub n_layers: c_int,
    pub max_seq: c_int,
    pub eps: f32,
}

// Opaque handles owned by the library.
#[repr(C)]
pub struct RkvBlockManager {
    _private: [u8; 0],
}
#[repr(C)]
pub struct RkvDeviceBlockManager {
    _private: [u8; 0],
}
#[repr(C)]
pub struct RkvScheduler {
    _private: [u8; 0],
}
#[repr(C)]
pub struct RkvDecoder {
    _private: [u8; 0],
}
#[repr(C)]
pub struct RkvEngine {
    _private: [u8; 0],
}
#[repr(C)]
pub struct RkvStFile {
    _private: [u8; 0],
}

#[link(name = "rustral_kv")]
extern "C" {
    // ---- include/rustral_kv.h
    pub fn rkv_last_error() -> *const c_char;
    pub fn rkv_version() -> c_int;
    pub fn rkv_append(
        k_pool: *mut c_void,
        v_pool: *mut c_void,
        pool_layer_stride: i64,
        k_new: *const f32,
        v_new: *const f32,
        src_layer_stride: i64,
        src_tok_stride: i64,
        src_head_stride: i64,
        slot_mapping: *const i64,
        n_tokens: i64,
        n_layers: c_int,
        num_kv_heads: c_int,
        head_dim: c_int,
        block_size: c_int,
        num_blocks: i64,
        dtype: c_int,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_gather(
        k_out: *mut c_void,
        v_out: *mut c_void,
        k_pool: *const c_void,
        v_pool: *const c_void,
        block_tables: *const i32,
        max_blocks_per_seq: c_int,
        ctx_lens: *const i32,
        out_offsets: *const i64,
        num_seqs: c_int,
        num_kv_heads: c_int,
        head_dim: c_int,
        block_size: c_int,
        num_blocks: i64,
        max_ctx: c_int,
        dtype: c_int,
        out_dtype: c_int,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_copy_blocks(
        k_pool: *mut c_void,
        v_pool: *mut c_void,
        layer_stride_bytes: i64,
        n_layers: c_int,
        pairs: *const i32,
        n_pairs: c_int,
        block_bytes: i64,
        num_blocks: i64,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_decode_workspace_bytes(
        num_seqs: c_int,
        num_q_heads: c_int,
        head_dim: c_int,
        max_context: c_int,
        partition_size: c_int,
    ) -> usize;
    pub fn rkv_decode_partition_size(
        partition_size: c_int,
        head_dim: c_int,
        dtype: c_int,
        max_context: c_int,
    ) -> c_int;
    pub fn rkv_decode_partition_size_for(
        partition_size: c_int,
        num_seqs: c_int,
        num_q_heads: c_int,
        num_kv_heads: c_int,
        head_dim: c_int,
        dtype: c_int,
        max_context: c_int,
    ) -> c_int;
    pub fn rkv_decode_attention(
        out: *mut f32,
        q: *const f32,
        k_pool: *const c_void,
        v_pool: *const c_void,
        block_tables: *const i32,
        max_blocks_per_seq: c_int,
        ctx_lens: *const i32,
        num_seqs: c_int,
        num_q_heads: c_int,
        num_kv_heads: c_int,
        head_dim: c_int,
        block_size: c_int,
        num_blocks: i64,
        max_context: c_int,
        scale: f32,
        dtype: c_int,
        partition_size: c_int,
        workspace: *mut c_void,
        workspace_bytes: usize,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_decode_attention_append(
        out: *mut f32,
        q: *const f32,
        k_pool: *mut c_void,
        v_pool: *mut c_void,
        k_new: *const f32,
        v_new: *const f32,
        block_tables: *const i32,
        max_blocks_per_seq: c_int,
        ctx_lens: *const i32,
        num_seqs: c_int,
        num_q_heads: c_int,
        num_kv_heads: c_int,
        head_dim: c_int,
        block_size: c_int,
        num_blocks: i64,
        max_context: c_int,
        scale: f32,
        dtype: c_int,
        partition_size: c_int,
        workspace: *mut c_void,
        workspace_bytes: usize,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_decode_attention_noalloc(
        out: *mut f32,
        q: *const f32,
        k_pool: *const c_void,
        v_pool: *const c_void,
        block_tables: *const i32,
        max_blocks_per_seq: c_int,
        ctx_lens: *const i32,
        num_seqs: c_int,
        num_q_heads: c_int,
        num_kv_heads: c_int,
        head_dim: c_int,
        block_size: c_int,
        num_blocks: i64,
        max_context: c_int,
        scale: f32,
        dtype: c_int,
        partition_size: c_int,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_decode_noalloc_max_bytes() -> usize;
    pub fn rkv_decode_attention_partitions(
        out: *mut f32,
        q: *const f32,
        k_pool: *const c_void,
        v_pool: *const c_void,
        block_tables: *const i32,
        max_blocks_per_seq: c_int,
        ctx_lens: *const i32,
        num_seqs: c_int,
        num_q_heads: c_int,
        num_kv_heads: c_int,
        head_dim: c_int,
        block_size: c_int,
        num_blocks: i64,
        max_context: c_int,
        scale: f32,
        dtype: c_int,
        partition_size: c_int,
        workspace: *mut c_void,
        workspace_bytes: usize,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_decode_attention_merge(
        out: *mut f32,
        ctx_lens: *const i32,
        max_blocks_per_seq: c_int,
        num_seqs: c_int,
        num_q_heads: c_int,
        head_dim: c_int,
        block_size: c_int,
        max_context: c_int,
        dtype: c_int,
        partition_size: c_int,
        workspace: *const c_void,
        workspace_bytes: usize,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_append_q(
        k_pool: *mut c_void,
        v_pool: *mut c_void,
        k_scale: *mut f32,
        v_scale: *mut f32,
        pool_layer_stride: i64,
        k_new: *const f32,
        v_new: *const f32,
        src_layer_stride: i64,
        src_tok_stride: i64,
        src_head_stride: i64,
        slot_mapping: *const i64,
        n_tokens: i64,
        n_layers: c_int,
        num_kv_heads: c_int,
        head_dim: c_int,
        block_size: c_int,
        num_blocks: i64,
        dtype: c_int,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_gather_q(
        k_out: *mut f32,
        v_out: *mut f32,
        k_pool: *const c_void,
        v_pool: *const c_void,
        k_scale: *const f32,
        v_scale: *const f32,
        block_tables: *const i32,
        max_blocks_per_seq: c_int,
        ctx_lens: *const i32,
        out_offsets: *const i64,
        num_seqs: c_int,
        num_kv_heads: c_int,
        head_dim: c_int,
        block_size: c_int,
        num_blocks: i64,
        max_ctx: c_int,
        dtype: c_int,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_decode_attention_q(
        out: *mut f32,
        q: *const f32,
        k_pool: *const c_void,
        v_pool: *const c_void,
        k_scale: *const f32,
        v_scale: *const f32,
        block_tables: *const i32,
        max_blocks_per_seq: c_int,
        ctx_lens: *const i32,
        num_seqs: c_int,
        num_q_heads: c_int,
        num_kv_heads: c_int,
        head_dim: c_int,
        block_size: c_int,
        num_blocks: i64,
        max_context: c_int,
        scale: f32,
        dtype: c_int,
        partition_size: c_int,
        workspace: *mut c_void,
        workspace_bytes: usize,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_decode_attention_append_q(
        out: *mut f32,
        q: *const f32,
        k_pool: *mut c_void,
        v_pool: *mut c_void,
        k_scale: *mut f32,
        v_scale: *mut f32,
        k_new: *const f32,
        v_new: *const f32,
        block_tables: *const i32,
        max_blocks_per_seq: c_int,
        ctx_lens: *const i32,
        num_seqs: c_int,
        num_q_heads: c_int,
        num_kv_heads: c_int,
        head_dim: c_int,
        block_size: c_int,
        num_blocks: i64,
        max_context: c_int,
        scale: f32,
        dtype: c_int,
        partition_size: c_int,
        workspace: *mut c_void,
        workspace_bytes: usize,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_prefill_attention(
        out: *mut f32,
        q: *const f32,
        k_pool: *const c_void,
        v_pool: *const c_void,
        block_tables: *const i32,
        max_blocks_per_seq: c_int,
        q_start: *const i32,
        ctx_lens: *const i32,
        num_seqs: c_int,
        num_q_heads: c_int,
        num_kv_heads: c_int,
        head_dim: c_int,
        block_size: c_int,
        num_blocks: i64,
        max_q_len: c_int,
        scale: f32,
        dtype: c_int,
        stream: Stream,
    ) -> c_int;
    // ---- include/rustral_model.h
    pub fn rkv_embed(
        out: *mut f32,
        table: *const f32,
        ids: *const i32,
        pe: *const f32,
        positions: *const i32,
        n_tokens: c_int,
        vocab: c_int,
        dim: c_int,
        max_len: c_int,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_linear(
        y: *mut f32,
        x: *const f32,
        w: *const f32,
        b: *const f32,
        rows: c_int,
        in_dim: c_int,
        out_dim: c_int,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_layer_norm(
        y: *mut f32,
        x: *const f32,
        g: *const f32,
        b: *const f32,
        rows: c_int,
        dim: c_int,
        eps: f32,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_qkv_append(
        q_out: *mut f32,
        k_pool: *mut c_void,
        v_pool: *mut c_void,
        slot_mapping: *const i64,
        x: *const f32,
        ln_g: *const f32,
        ln_b: *const f32,
        eps: f32,
        wq: *const f32,
        bq: *const f32,
        wk: *const f32,
        bk: *const f32,
        wv: *const f32,
        bv: *const f32,
        n_tokens: c_int,
        d_model: c_int,
        q_dim: c_int,
        num_kv_heads: c_int,
        head_dim: c_int,
        block_size: c_int,
        num_blocks: i64,
        dtype: c_int,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_gelu(y: *mut f32, x: *const f32, n: i64, stream: Stream) -> c_int;
    pub fn rkv_add(y: *mut f32, a: *const f32, b: *const f32, n: i64, stream: Stream) -> c_int;
    pub fn rkv_mul_scalar(y: *mut f32, x: *const f32, s: f32, n: i64, stream: Stream) -> c_int;
    pub fn rkv_softmax_dim(y: *mut f32, x: *const f32, outer: i64, axis: i64, inner: i64, stream: Stream) -> c_int;
    pub fn rkv_matmul(y: *mut f32, a: *const f32, b: *const f32, m: c_int, k: c_int, n: c_int, stream: Stream)
        -> c_int;
    pub fn rkv_transpose(y: *mut f32, x: *const f32, m: c_int, n: c_int, stream: Stream) -> c_int;
    pub fn rkv_argmax(out: *mut i32, x: *const f32, rows: c_int, n: c_int, stream: Stream) -> c_int;
    pub fn rkv_decoder_param_count(cfg: *const RkvDecoderConfig) -> i64;
    pub fn rkv_decoder_init_params(
        cfg: *const RkvDecoderConfig,
        seed: u64,
        std: f32,
        host_params: *mut f32,
    ) -> c_int;
    pub fn rkv_decoder_create(
        cfg: *const RkvDecoderConfig,
        host_params: *const f32,
        n_params: i64,
        stream: Stream,
    ) -> *mut RkvDecoder;
    pub fn rkv_decoder_destroy(dec: *mut RkvDecoder);
    pub fn rkv_decoder_generate(
        dec: *mut RkvDecoder,
        prompt: *const i32,
        n_prompt: c_int,
        n_new: c_int,
        out_tokens: *mut i32,
        out_logits: *mut f32,
    ) -> c_int;
    pub fn rkv_decoder_load_safetensors(
        cfg: *const RkvDecoderConfig,
        path: *const c_char,
        host_params: *mut f32,
        n_params: i64,
    ) -> c_int;
    pub fn rkv_decoder_save_safetensors(
        cfg: *const RkvDecoderConfig,
        host_params: *const f32,
        n_params: i64,
        path: *const c_char,
    ) -> c_int;
    pub fn rkv_decoder_load_safetensors_device(dec: *mut RkvDecoder, path: *const c_char) -> c_int;
    pub fn rkv_decoder_create_from_safetensors(
        cfg: *const RkvDecoderConfig,
        path: *const c_char,
        stream: Stream,
    ) -> *mut RkvDecoder;
    pub fn rkv_st_open(path: *const c_char) -> *mut RkvStFile;
    pub fn rkv_st_close(f: *mut RkvStFile);
    pub fn rkv_st_num_tensors(f: *const RkvStFile) -> i64;
    pub fn rkv_st_tensor(
        f: *const RkvStFile,
        i: i64,
        name: *mut *const c_char,
        dtype: *mut *const c_char,
        ndim: *mut c_int,
        shape: *mut i64,
        max_dims: c_int,
    ) -> c_int;
    pub fn rkv_st_load(
        f: *const RkvStFile,
        n: c_int,
        names: *const *const c_char,
        ndims: *const c_int,
        shapes: *const i64,
        dsts: *const *mut c_void,
        dst_on_device: c_int,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_engine_create(
        cfg: *const RkvDecoderConfig,
        host_params: *const f32,
        n_params: i64,
        num_blocks: i64,
        max_batch_size: c_int,
        stream: Stream,
    ) -> *mut RkvEngine;
    pub fn rkv_engine_destroy(e: *mut RkvEngine);
    pub fn rkv_engine_submit(
        e: *mut RkvEngine,
        prompt: *const i32,
        n_prompt: c_int,
        max_tokens: c_int,
        priority: c_int,
    ) -> i64;
    pub fn rkv_engine_step(e: *mut RkvEngine) -> c_int;
    pub fn rkv_engine_run(e: *mut RkvEngine, max_steps: c_int) -> c_int;
    pub fn rkv_engine_scheduler(e: *mut RkvEngine) -> *mut RkvScheduler;
    pub fn rkv_rng_raw(seed: u64, out: *mut u64, n: i64) -> c_int;
    pub fn rkv_fill_normal(out: *mut f32, n: i64, seed: u64, std: f32) -> c_int;
    // ---- include/rustral_serving.h
    pub fn rkv_bm_create(num_blocks: i64, block_size: c_int) -> *mut RkvBlockManager;
    pub fn rkv_bm_destroy(bm: *mut RkvBlockManager);
    pub fn rkv_bm_allocate(
        bm: *mut RkvBlockManager,
        seq_id: i64,
        num_tokens: i64,
        out_ids: *mut i32,
        cap: i64,
    ) -> i64;
    pub fn rkv_bm_reserve(bm: *mut RkvBlockManager, seq_id: i64, num_tokens: i64) -> i64;
    pub fn rkv_bm_free(bm: *mut RkvBlockManager, seq_id: i64) -> i64;
    pub fn rkv_bm_num_free(bm: *const RkvBlockManager) -> i64;
    pub fn rkv_bm_num_blocks(bm: *const RkvBlockManager) -> i64;
    pub fn rkv_bm_block_size(bm: *const RkvBlockManager) -> c_int;
    pub fn rkv_bm_table(bm: *const RkvBlockManager, seq_id: i64, out: *mut i32, cap: i64) -> i64;
    pub fn rkv_bm_free_list(bm: *const RkvBlockManager, out: *mut i32, cap: i64) -> i64;
    pub fn rkv_bm_fill_tables(
        bm: *const RkvBlockManager,
        seq_ids: *const i64,
        n_seqs: c_int,
        tables: *mut i32,
        max_blocks: c_int,
    ) -> c_int;
    pub fn rkv_bm_plan_compaction(
        bm: *mut RkvBlockManager,
        max_moves: i64,
        pairs: *mut i32,
        cap_pairs: i64,
    ) -> i64;
    pub fn rkv_bm_plan_migration(
        bm: *mut RkvBlockManager,
        max_moves: i64,
        pairs: *mut i32,
        cap_pairs: i64,
    ) -> i64;
    pub fn rkv_bm_plan_relocation(
        bm: *mut RkvBlockManager,
        max_moves: i64,
        pairs: *mut i32,
        cap_pairs: i64,
    ) -> i64;
    pub fn rkv_dbm_create(
        num_blocks: i64,
        block_size: c_int,
        max_seqs: c_int,
        max_blocks_per_seq: c_int,
        stream: Stream,
    ) -> *mut RkvDeviceBlockManager;
    pub fn rkv_dbm_destroy(bm: *mut RkvDeviceBlockManager);
    pub fn rkv_dbm_reserve(
        bm: *mut RkvDeviceBlockManager,
        slots: *const i32,
        num_tokens: *const i32,
        n: c_int,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_dbm_free(
        bm: *mut RkvDeviceBlockManager,
        slots: *const i32,
        n: c_int,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_dbm_slot_mapping(
        bm: *const RkvDeviceBlockManager,
        slots: *const i32,
        positions: *const i32,
        n: c_int,
        slot_mapping: *mut i64,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_dbm_batch_tables(
        bm: *const RkvDeviceBlockManager,
        slots: *const i32,
        n: c_int,
        tables: *mut i32,
        max_blocks: c_int,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_dbm_status(
        bm: *mut RkvDeviceBlockManager,
        num_free: *mut i64,
        err: *mut i32,
        clear: c_int,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_dbm_download(
        bm: *const RkvDeviceBlockManager,
        tables: *mut i32,
        lengths: *mut i32,
        free_list: *mut i32,
        num_free: *mut i64,
        stream: Stream,
    ) -> c_int;
    pub fn rkv_sched_create(
        num_blocks: i64,
        block_size: c_int,
        max_batch_size: c_int,
        max_seq_len: c_int,
    ) -> *mut RkvScheduler;
    pub fn rkv_sched_destroy(s: *mut RkvScheduler);
    pub fn rkv_sched_add_request(
        s: *mut RkvScheduler,
        prompt: *const i32,
        n_prompt: c_int,
        max_tokens: c_int,
        priority: c_int,
    ) -> i64;
    pub fn rkv_sched_schedule(s: *mut RkvScheduler) -> c_int;
    pub fn rkv_sched_batch_dims(
        s: *const RkvScheduler,
        n_requests: *mut c_int,
        n_input_tokens: *mut i64,
        max_blocks: *mut c_int,
    ) -> c_int;
    pub fn rkv_sched_batch(
        s: *const RkvScheduler,
        request_ids: *mut i64,
        seq_lens: *mut i32,
        input_offsets: *mut i64,
        input_ids: *mut i32,
        positions: *mut i32,
        block_tables: *mut i32,
        max_blocks: c_int,
    ) -> c_int;
    pub fn rkv_sched_update(
        s: *mut RkvScheduler,
        request_ids: *const i64,
        tokens: *const i32,
        n: c_int,
    ) -> c_int;
    pub fn rkv_sched_stats(s: *const RkvScheduler, out5: *mut i64) -> c_int;
    pub fn rkv_sched_generated(
        s: *const RkvScheduler,
        request_id: i64,
        out: *mut i32,
        cap: i64,
    ) -> i64;
    pub fn rkv_sched_block_manager(s: *mut RkvScheduler) -> *mut RkvBlockManager;
    pub fn rkv_sampler_greedy(logits: *const f32, n: c_int) -> c_int;
}

/// The HIP runtime calls the backend needs for device memory and its stream
/// (libamdhip64).
pub mod hip {
    use std::os::raw::{c_int, c_void};
    pub type HipError = c_int;
    pub const HIP_SUCCESS: HipError = 0;
    pub const HIP_MEMCPY_HOST_TO_DEVICE: c_int = 1;
    pub const HIP_MEMCPY_DEVICE_TO_HOST: c_int = 2;
    pub const HIP_MEMCPY_DEVICE_TO_DEVICE: c_int = 3;
    pub const HIP_STREAM_NON_BLOCKING: u32 = 1;

    #[link(name = "amdhip64")]
    extern "C" {
        pub fn hipSetDevice(device: c_int) -> HipError;
        pub fn hipGetDeviceCount(count: *mut c_int) -> HipError;
        pub fn hipMalloc(ptr: *mut *mut c_void, size: usize) -> HipError;
        pub fn hipFree(ptr: *mut c_void) -> HipError;
        pub fn hipMemcpyAsync(
            dst: *mut c_void,
            src: *const c_void,
            size: usize,
            kind: c_int,
            stream: *mut c_void,
        ) -> HipError;
        pub fn hipMemsetAsync(dst: *mut c_void, value: c_int, size: usize, stream: *mut c_void)
            -> HipError;
        pub fn hipStreamCreateWithFlags(stream: *mut *mut c_void, flags: u32) -> HipError;
        pub fn hipStreamDestroy(stream: *mut c_void) -> HipError;
        pub fn hipStreamSynchronize(stream: *mut c_void) -> HipError;
        pub fn hipGetErrorString(err: HipError) -> *const std::os::raw::c_char;
    }
}
