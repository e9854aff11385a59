/*
 * rustral_kv.h -- C ABI of the MI355X (gfx950) paged-KV library
 * librustral_kv.so.
 *
 * This is the drop-in boundary under rustral's KV-cache and attention
 * interfaces.  rustral's own CPU path for these operations is a stub
 * (crates/nn/src/kv_cache.rs:172-243, :381-432); each entry point below
 * names the reference interface it stands in for.
 *
 * Conventions shared by every entry point
 *  - All pointers are DEVICE pointers unless marked "host".  Nothing is
 *    freed or kept: the caller owns every buffer.
 *  - stream: an opaque hipStream_t (NULL = the default stream).  Work is
 *    enqueued asynchronously; nothing synchronizes.
 *  - Return value: RKV_OK (0) or a negative RKV_ERR_* code.  The message of
 *    the last failure on the calling thread is rkv_last_error().  Argument
 *    errors are detected on the host before any launch.  Entries the host
 *    cannot see (block ids, slots, context lengths) are range-checked on the
 *    device and out-of-range entries are skipped, never dereferenced.
 *  - KV pool layout, one pool per layer and per K/V:
 *        pool[num_blocks][num_kv_heads][block_size][head_dim]
 *    dtype RKV_F32 (float) or RKV_BF16 (bf16 bits; fp32 -> bf16 rounds to
 *    nearest even, NaN stays NaN).  Token position p of a sequence is row
 *    p % block_size of block block_table[p / block_size].
 *  - GQA: query head h reads KV head h / (num_q_heads / num_kv_heads).
 *  - Supported shapes: head_dim in {32, 64, 128}, block_size 16,
 *    num_q_heads / num_kv_heads in {1, 2, 4, 8} (append/gather/copy accept
 *    any head_dim that is a multiple of 8).
 */
#ifndef RUSTRAL_KV_H
#define RUSTRAL_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RKV_F32 0
#define RKV_BF16 1
#define RKV_I8 2  /* int8 bytes + one fp32 scale per (token, KV head) row   */
#define RKV_FP8 3 /* OCP fp8 e4m3 bytes + one fp32 scale per row            */

#define RKV_OK 0
#define RKV_ERR_INVALID_ARG (-1) /* maps to CoreError::InvalidArgument / Shape */
#define RKV_ERR_UNSUPPORTED (-2) /* shape/dtype combination not built     */
#define RKV_ERR_WORKSPACE (-3)   /* workspace missing or too small         */
#define RKV_ERR_HIP (-4)         /* HIP launch/runtime error -> Backend(msg) */

/* Thread-local message of the last failed call ("" if none).  Stands in for
 * the String payload of CoreError (crates/core/src/error.rs:8-46). */
const char* rkv_last_error(void);

/* ABI version, major*10000 + minor*100 + patch. */
int rkv_version(void);

/* Append new K/V rows into paged pools.
 * Replaces KVCache::append (crates/nn/src/kv_cache.rs:172-216), which
 * intends to write new_k/new_v [batch, Hkv, T, D] at positions
 * current_len..current_len+T but writes nothing.
 *
 * For layer l < n_layers, token t < n_tokens, head h, dim d:
 *   src = k_new + l*src_layer_stride + t*src_tok_stride + h*src_head_stride + d
 *   dst = k_pool + l*pool_layer_stride + ((blk*Hkv + h)*block_size + row)*head_dim + d
 * with slot_mapping[t] = blk*block_size + row (int64, shared by all layers).
 * Strides are in elements; src strides must be multiples of 4 and src
 * pointers 16-byte aligned.  Slots < 0 (padding) or >= num_blocks*block_size
 * are skipped.  One launch covers every layer. */
int rkv_append(void* k_pool, void* v_pool, int64_t pool_layer_stride, const float* k_new,
               const float* v_new, int64_t src_layer_stride, int64_t src_tok_stride,
               int64_t src_head_stride, const int64_t* slot_mapping, int64_t n_tokens,
               int n_layers, int num_kv_heads, int head_dim, int block_size,
               int64_t num_blocks, int dtype, void* stream);

/* Gather each sequence's K/V into the contiguous KVCache layout.
 * Replaces KVCache::get_range / k_cache / v_cache
 * (crates/nn/src/kv_cache.rs:219-243), whose layout is
 * [batch, Hkv, seq, D] (kv_cache.rs:139-142).
 * Sequence b (L_b = ctx_lens[b], clamped to max_blocks_per_seq*block_size)
 * is written to
 *   out_offsets == NULL: out[b][h][p][d] with shape [num_seqs, Hkv, max_ctx, D]
 *                        (rejected on the device side if L_b > max_ctx: rows
 *                        p >= max_ctx are not written)
 *   out_offsets != NULL: out + out_offsets[b] + (h*L_b + p)*D + d  (packed)
 * Only tokens p < L_b are written.  out_dtype is dtype (bit copy) or RKV_F32
 * (exact bf16 -> fp32 upcast).  Blocks with an id outside [0, num_blocks)
 * are skipped. */
int rkv_gather(void* k_out, void* v_out, const void* k_pool, const void* v_pool,
               const int32_t* block_tables, int max_blocks_per_seq, const int32_t* ctx_lens,
               const int64_t* out_offsets, int num_seqs, int num_kv_heads, int head_dim,
               int block_size, int64_t num_blocks, int max_ctx, int dtype, int out_dtype,
               void* stream);

/* Copy whole blocks (all heads, all rows) inside every layer's K and V pool:
 * for l < n_layers, i < n_pairs: block pairs[2i+1] := block pairs[2i].
 * No reference counterpart: PagedCache only allocates and frees block ids
 * (crates/nn/src/kv_cache.rs:413-431) and eviction is a free
 * (crates/nn/src/continuous_batching.rs:380-386).  This is the compaction
 * step of continuous batching.  block_bytes = Hkv*block_size*head_dim*elem
 * (multiple of 16); layer l's pool starts at pool + l*layer_stride_bytes.
 * The set of destinations must not intersect the set of sources within one
 * call (results are then independent of execution order). */
int rkv_copy_blocks(void* k_pool, void* v_pool, int64_t layer_stride_bytes, int n_layers,
                    const int32_t* pairs, int n_pairs, int64_t block_bytes, int64_t num_blocks,
                    void* stream);

/* Workspace (bytes) rkv_decode_attention needs for split-K partials.
 * max_context: host-side upper bound on every ctx_lens[b] (for example
 * max_blocks_per_seq*block_size).  partition_size: the size the call will
 * use (rkv_decode_partition_size_for), or <= 0 for the smallest size any
 * call picks by itself (512), which is enough for every pool dtype and
 * shape. */
size_t rkv_decode_workspace_bytes(int num_seqs, int num_q_heads, int head_dim, int max_context,
                                  int partition_size);

/* Partition size (tokens) for pools of dtype and this max_context, for a
 * request of partition_size: the request itself when it is a multiple of 64
 * tokens (16 tokens x 4 waves) up to 640, or for RKV_BF16 pools a multiple
 * of 128 (16 tokens x 8 waves) up to 1280; for partition_size <= 0 the size
 * the split entry points (rkv_decode_attention_partitions / _merge) use,
 * 640.  RKV_ERR_UNSUPPORTED for other requests.  What rkv_decode_attention
 * picks for a whole call: rkv_decode_partition_size_for. */
int rkv_decode_partition_size(int partition_size, int head_dim, int dtype, int max_context);

/* Partition size rkv_decode_attention (and _noalloc) uses for a call of this
 * shape: the request when partition_size > 0 (rules of
 * rkv_decode_partition_size), else its own pick.  With W = num_kv_heads *
 * num_seqs * max_context / 2 tokens: RKV_F32 and RKV_BF16 pools take 512
 * when W < 800 * 512, 1-byte pools when W < 1600 * 512; above that, RKV_BF16
 * pools with head_dim 128 and at most 4 query heads per KV head take 1280
 * when W >= 1200 * 1280, else 768 when W >= 1000 * 768, else 640; every
 * other shape and dtype 640.  The split entry points take this value as their
 * partition_size to match the one-call entry point. */
int rkv_decode_partition_size_for(int partition_size, int num_seqs, int num_q_heads,
                                  int num_kv_heads, int head_dim, int dtype, int max_context);

/* Single-token paged decode attention with GQA (two passes: partitions of
 * partition_size tokens -- see rkv_decode_partition_size; <= 0 for the
 * library's pick for this shape, rkv_decode_partition_size_for -- then a
 * merge; one partition skips the merge).
 * Replaces the per-head recipe of TapeMultiHeadAttention
 * (crates/nn/src/tape_transformer.rs:87-139), for one query token per
 * sequence attending to its whole cache, and AttentionOps
 * (crates/core/src/backend.rs:551-602), which has no block tables.
 *   out[b][h][:] = softmax_j((q[b][h] . K[b][kv(h)][j]) * scale) @ V[b][kv(h)][j]
 * q, out: [num_seqs, num_q_heads, head_dim] fp32.  Accumulation is fp32.
 * block_tables: [num_seqs, max_blocks_per_seq] int32; ctx_lens: [num_seqs].
 * L_b <= 0 gives a zero row.  max_context is the host-side upper bound used
 * to size the grid (<= max_blocks_per_seq*block_size).
 * workspace: >= rkv_decode_workspace_bytes(...) bytes, may be NULL when
 * max_context <= partition size. */
int rkv_decode_attention(float* out, const float* q, const void* k_pool, const void* v_pool,
                         const int32_t* block_tables, int max_blocks_per_seq,
                         const int32_t* ctx_lens, int num_seqs, int num_q_heads,
                         int num_kv_heads, int head_dim, int block_size, int64_t num_blocks,
                         int max_context, float scale, int dtype, int partition_size,
                         void* workspace, size_t workspace_bytes, void* stream);

/* One decode step's K/V append fused into rkv_decode_attention (RKV_BF16
 * pools, else RKV_ERR_UNSUPPORTED; 1-byte pools: rkv_decode_attention_append_q).  Replaces the pair a decode step
 * makes per layer, KVCache::append (crates/nn/src/kv_cache.rs:172-216) of the
 * step's one token, then the attention over the cache
 * (crates/nn/src/tape_transformer.rs:87-139).  ctx_lens[b] already counts
 * the new token: its K/V rows k_new/v_new [num_seqs][num_kv_heads][head_dim]
 * fp32 (16-byte aligned) go to position ctx_lens[b] - 1, i.e. slot
 * block_tables[b][(L-1)/16]*16 + (L-1)%16, rounded to bf16 as rkv_append
 * rounds them; a block id outside [0, num_blocks) is not written, nor is the
 * row of a sequence whose ctx_lens[b] exceeds the context cap (max_context,
 * max_blocks_per_seq*block_size).  Pools and out afterwards equal rkv_append
 * of those rows followed by rkv_decode_attention, bit for bit.  The new
 * token's block must not be shared with another sequence of the call (a
 * block being appended to is never shared in a copy-on-write cache).  Other
 * arguments as rkv_decode_attention. */
int rkv_decode_attention_append(float* out, const float* q, void* k_pool, void* v_pool,
                                const float* k_new, const float* v_new,
                                const int32_t* block_tables, int max_blocks_per_seq,
                                const int32_t* ctx_lens, int num_seqs, int num_q_heads,
                                int num_kv_heads, int head_dim, int block_size,
                                int64_t num_blocks, int max_context, float scale, int dtype,
                                int partition_size, void* workspace, size_t workspace_bytes,
                                void* stream);

/* rkv_decode_attention without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference: its
 * attention allocates freely.  The split-K partials live in a 16 MiB array
 * the library keeps on each GPU it runs on (rkv_decode_noalloc_max_bytes());
 * a call whose partials (rkv_decode_workspace_bytes) exceed it fails with
 * RKV_ERR_WORKSPACE.  The call allocates nothing: no hipMalloc, no library
 * allocator.  The array is shared by every call on one GPU and keeps the
 * last call's contents, so calls that overlap on one GPU (concurrent streams
 * or threads) race; serialise them on one stream.  Same arguments and result
 * as rkv_decode_attention otherwise. */
int rkv_decode_attention_noalloc(float* out, const float* q, const void* k_pool,
                                 const void* v_pool, const int32_t* block_tables,
                                 int max_blocks_per_seq, const int32_t* ctx_lens, int num_seqs,
                                 int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                 int64_t num_blocks, int max_context, float scale, int dtype,
                                 int partition_size, void* stream);

/* Size in bytes of the per-GPU scratch of rkv_decode_attention_noalloc. */
size_t rkv_decode_noalloc_max_bytes(void);

/* The two passes of rkv_decode_attention as separate launches, for callers
 * that schedule them apart (and for per-kernel timing).  Same arguments;
 * pass 1 writes finished rows for single-partition sequences and partials
 * for the rest, pass 2 merges the partials.  Both passes must be given the
 * same partition_size; <= 0 means 640 here (the merge has no KV-head count
 * to pick by shape), so to match rkv_decode_attention pass the value of
 * rkv_decode_partition_size_for. */
int rkv_decode_attention_partitions(float* out, const float* q, const void* k_pool,
                                    const void* v_pool, const int32_t* block_tables,
                                    int max_blocks_per_seq, const int32_t* ctx_lens,
                                    int num_seqs, int num_q_heads, int num_kv_heads,
                                    int head_dim, int block_size, int64_t num_blocks,
                                    int max_context, float scale, int dtype,
                                    int partition_size, void* workspace,
                                    size_t workspace_bytes, void* stream);
int rkv_decode_attention_merge(float* out, const int32_t* ctx_lens, int max_blocks_per_seq,
                               int num_seqs, int num_q_heads, int head_dim, int block_size,
                               int max_context, int dtype, int partition_size,
                               const void* workspace, size_t workspace_bytes, void* stream);

/* ---- 1-byte pools (CacheQuantization::Int8 / Fp8) ---------------------------
 * The reference lists these modes (crates/nn/src/kv_cache.rs:38-63) but its
 * quantize_kv (:266-296) scales twice (x / s * 127, then clamped) and its
 * dequantize_kv (:299-314) is never called, so the format is this library's:
 * each row -- the head_dim values of one token of one KV head -- is stored as
 * head_dim bytes in a pool laid out like the others ([num_blocks][Hkv]
 * [block_size][head_dim] uint8) plus one fp32 scale in a scale pool
 * [num_blocks][Hkv][block_size]:
 *   RKV_I8:  s = max|x| / 127, byte = rint(x * (127 / max|x|)) clamped to
 *            [-127, 127] (int8; max|x| = 0 or NaN input: 0); value = byte * s.
 *   RKV_FP8: s = max|x| / 448, byte = OCP e4m3 of x * (448 / max|x|), round to
 *            nearest even, magnitudes >= 448 saturating to 448; value =
 *            e4m3(byte) * s.
 * Compaction of 1-byte pools calls rkv_copy_blocks twice: on the byte pools
 * (block_bytes = Hkv*block_size*head_dim) and on the scale pools (block_bytes
 * = Hkv*block_size*4). */

/* rkv_append for 1-byte pools: quantizes each appended (token, head) row and
 * writes its bytes and scale.  Same arguments as rkv_append plus the scale
 * pools; pool_layer_stride is in bytes (= elements) of the byte pools, the
 * scale pools' layer stride is pool_layer_stride / head_dim.  head_dim 32, 64
 * or 128. */
int rkv_append_q(void* k_pool, void* v_pool, float* k_scale, float* v_scale,
                 int64_t pool_layer_stride, const float* k_new, const float* v_new,
                 int64_t src_layer_stride, int64_t src_tok_stride, int64_t src_head_stride,
                 const int64_t* slot_mapping, int64_t n_tokens, int n_layers, int num_kv_heads,
                 int head_dim, int block_size, int64_t num_blocks, int dtype, void* stream);

/* rkv_gather for 1-byte pools: dequantized fp32 output (byte value * row
 * scale) in the same padded or packed layouts. */
int rkv_gather_q(float* k_out, float* v_out, const void* k_pool, const void* v_pool,
                 const float* k_scale, const float* v_scale, const int32_t* block_tables,
                 int max_blocks_per_seq, const int32_t* ctx_lens, const int64_t* out_offsets,
                 int num_seqs, int num_kv_heads, int head_dim, int block_size,
                 int64_t num_blocks, int max_ctx, int dtype, void* stream);

/* rkv_decode_attention over 1-byte pools: the same result as decode on the
 * dequantized values (scores = (q . bytes) * scale * row scale; the V row
 * scale multiplies the softmax weight).  head_dim 64 or 128; workspace as
 * rkv_decode_workspace_bytes. */
int rkv_decode_attention_q(float* out, const float* q, const void* k_pool, const void* v_pool,
                           const float* k_scale, const float* v_scale,
                           const int32_t* block_tables, int max_blocks_per_seq,
                           const int32_t* ctx_lens, int num_seqs, int num_q_heads,
                           int num_kv_heads, int head_dim, int block_size, int64_t num_blocks,
                           int max_context, float scale, int dtype, int partition_size,
                           void* workspace, size_t workspace_bytes, void* stream);

/* rkv_decode_attention_append for 1-byte pools (RKV_I8 / RKV_FP8): the new
 * rows are quantized as rkv_append_q quantizes them (bytes and row scale);
 * pools, scale pools and out equal rkv_append_q followed by
 * rkv_decode_attention_q, bit for bit.  Replaces the same pair of reference
 * calls as rkv_decode_attention_append (crates/nn/src/kv_cache.rs:172-216,
 * crates/nn/src/tape_transformer.rs:87-139) for a cache whose
 * CacheConfig::quantization (kv_cache.rs:38-63) is Int8 or Fp8.  Other
 * arguments as rkv_decode_attention_q. */
int rkv_decode_attention_append_q(float* out, const float* q, void* k_pool, void* v_pool,
                                  float* k_scale, float* v_scale, const float* k_new,
                                  const float* v_new, const int32_t* block_tables,
                                  int max_blocks_per_seq, const int32_t* ctx_lens, int num_seqs,
                                  int num_q_heads, int num_kv_heads, int head_dim,
                                  int block_size, int64_t num_blocks, int max_context,
                                  float scale, int dtype, int partition_size, void* workspace,
                                  size_t workspace_bytes, void* stream);

/* Causal prefill attention over the paged pool (many new query tokens per
 * sequence).  Sequence b owns query rows q_start[b] .. q_start[b+1]-1 of q
 * and out ([total, num_q_heads, head_dim] fp32, total = q_start[num_seqs]);
 * its n_b new tokens are the last n_b of its ctx_lens[b] cached tokens (their
 * K/V appended beforehand with rkv_append), so new token i sits at position
 * p = ctx_lens[b] - n_b + i and attends to positions 0 .. p:
 *   out[row][h][:] = softmax_{j<=p}((q[row][h] . K[b][kv(h)][j]) * scale) @ V
 * Replaces the per-head recipe of TapeMultiHeadAttention::forward_tape_with_mask
 * (crates/nn/src/tape_transformer.rs:87-139) with the additive causal mask of
 * causal_mask_tape (:276-296; -1e9 above the diagonal gives a zero weight),
 * reading K/V through block tables; ctx_lens[b] == n_b is the reference's
 * square case, a larger ctx_lens[b] a chunked prefill after cached tokens.
 * max_q_len: host-side bound on the n_b (it sizes the grid); only the first
 * max_q_len new tokens of a sequence are computed, later rows are not
 * written.  Rows with p < 0 are zero; positions at or beyond
 * max_blocks_per_seq*block_size and blocks with an invalid id are left out.
 * block_size 16; head_dim 32, 64 or 128; num_q_heads / num_kv_heads 1, 2, 4
 * or 8.  No workspace. */
int rkv_prefill_attention(float* out, const float* q, const void* k_pool, const void* v_pool,
                          const int32_t* block_tables, int max_blocks_per_seq,
                          const int32_t* q_start, const int32_t* ctx_lens, int num_seqs,
                          int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                          int64_t num_blocks, int max_q_len, float scale, int dtype,
                          void* stream);

#ifdef __cplusplus
}
#endif
#endif /* RUSTRAL_KV_H */
