/*
 * rkv_oracle.h -- CPU restatement of rustral's paged-KV hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or the timed CPU baseline).  The product path (rustral_amd,
 * librustral_kv.so) never links or calls it.
 *
 * rustral's own KV path cannot serve as the oracle: KVCache::append writes
 * nothing (crates/nn/src/kv_cache.rs:197-210), get_range returns the whole
 * cache (kv_cache.rs:229-243) and PagedCache has no storage
 * (kv_cache.rs:399-409).  This file restates what those functions are
 * documented to do, built from the ndarray primitive semantics the reference
 * composes attention from.  Each function cites the file:line it follows.
 *
 * Layout shared with the GPU library (one pool per layer, K and V separate):
 *     pool[num_blocks][num_kv_heads][block_size][head_dim]
 * Token position p of a sequence lives in block block_table[p / block_size]
 * at row p % block_size.  Query head h reads KV head h / (Hq / Hkv).
 *
 * How each function is pinned is listed in the tests (tests/test_oracle.py,
 * tests/test_model.py).
 */
#ifndef RKV_ORACLE_H
#define RKV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_BF16 = 1, ORC_I8 = 2, ORC_FP8 = 3 };

/* fp32 -> bf16 round-to-nearest-even, NaN kept as a quiet NaN of the same
 * sign.  Deviation from the reference's only converter, which truncates
 * (crates/distributed/src/compression.rs:256-261). */
uint16_t orc_bf16_from_f32(float x);
float orc_f32_from_bf16(uint16_t b);
void orc_bf16_from_f32_array(const float* x, uint16_t* y, int64_t n);
void orc_f32_from_bf16_array(const uint16_t* x, float* y, int64_t n);

/* KV append: the write KVCache::append intends (kv_cache.rs:172-216), into
 * a paged pool.  Token t (0 <= t < n_tokens) of source row
 * src[t*src_tok_stride + h*src_head_stride + d] goes to flat slot
 * slot_mapping[t] = block * block_size + row.  Slots < 0 (padding) or
 * >= num_blocks*block_size are skipped.  Returns 0, or -1 on bad args. */
int orc_append(void* k_pool, void* v_pool, const float* k_new, const float* v_new,
               const int64_t* slot_mapping, int64_t n_tokens, int num_kv_heads, int head_dim,
               int block_size, int64_t num_blocks, int64_t src_tok_stride,
               int64_t src_head_stride, int pool_dtype);

/* KV gather: the slice KVCache::get_range intends (kv_cache.rs:229-243),
 * reconstructed through block tables.  Sequence b's K (and V) are written in
 * the KVCache layout [Hkv, L_b, D] (kv_cache.rs:139-142) at
 *   out_offsets == NULL : out + (b*Hkv*max_ctx)   with row stride max_ctx
 *   out_offsets != NULL : out + out_offsets[b]    with row stride L_b
 * Only tokens < L_b are written; a block id outside [0, num_blocks) leaves
 * its 16 rows untouched.  out_dtype may be the pool dtype or F32 (exact
 * upcast of bf16). */
int orc_gather(void* k_out, void* v_out, const void* k_pool, const void* v_pool,
               const int32_t* block_tables, int max_blocks_per_seq, const int32_t* ctx_lens,
               const int64_t* out_offsets, int num_seqs, int num_kv_heads, int head_dim,
               int block_size, int64_t num_blocks, int max_ctx, int pool_dtype, int out_dtype);

/* Block copy for compaction: no reference function exists (PagedCache only
 * allocates/frees, kv_cache.rs:413-431).  For every layer l and pair i,
 * block pairs[2i+1] of layer l's pool becomes a copy of block pairs[2i].
 * Layer l's pool starts at pool + l*layer_stride_bytes.  Pairs with an id
 * outside [0, num_blocks) are skipped. */
int orc_copy_blocks(void* k_pool, void* v_pool, int64_t layer_stride_bytes, int n_layers,
                    const int32_t* pairs, int n_pairs, int64_t block_bytes, int64_t num_blocks);

/* Row softmax: CpuOps::softmax_dim on the last axis
 * (crates/ndarray-backend/src/lib.rs:1188-1227): max, exp(x-max), serial sum,
 * multiply by 1/sum. */
void orc_softmax_rows(const float* x, float* y, int rows, int cols);

/* CpuOps::softmax_dim on any axis of a tensor viewed as [outer][axis][inner]
 * (lib.rs:1188-1227); axis <= 0 -> -1 (the reference's InvalidArgument). */
int orc_softmax_dim(const float* x, float* y, int64_t outer, int64_t axis, int64_t inner);

/* CpuOps::matmul's naive order (lib.rs:208-219), rank 2, row-major. */
void orc_matmul(const float* a, const float* b, float* y, int m, int k, int n);

/* CpuOps::transpose (lib.rs:270-281), rank 2. */
void orc_transpose(const float* x, float* y, int m, int n);

/* CpuOps::mul_scalar (lib.rs:747-756). */
void orc_mul_scalar(const float* x, float* y, float s, int64_t n);

/* Greedy argmax: last index among equal maxima, as Iterator::max_by in
 * CpuOps::argmax (ndarray-backend/src/lib.rs:430-437) and Sampler::greedy
 * (crates/nn/src/continuous_batching.rs:458-462).  n == 0 -> -1. */
int64_t orc_argmax(const float* x, int64_t n);

/* Single-token decode attention over the paged pool, per (sequence b, query
 * head h), following TapeMultiHeadAttention::forward_tape_with_mask
 * (crates/nn/src/tape_transformer.rs:87-139) with ndarray op semantics:
 *   s_j = (q . k_j) * scale          matmul naive order (lib.rs:207-217),
 *                                    scale after the dot (attention.rs:127-134)
 *   p   = softmax_dim(s)             (lib.rs:1188-1227)
 *   o_d = sum_j p_j * v_j[d]         matmul naive order
 * j runs over 0 <= j < L_b (no mask: decode attends to every cached token).
 * L_b <= 0 gives a zero output; L_b is clamped to max_blocks_per_seq *
 * block_size; tokens in blocks with an id outside [0, num_blocks) are left
 * out of the softmax.  q and out are [B, Hq, D] fp32. */
int orc_decode_attention(float* out, const float* q, const void* k_pool, const void* v_pool,
                         const int32_t* block_tables, int max_blocks_per_seq,
                         const int32_t* ctx_lens, int num_seqs, int num_q_heads, int num_kv_heads,
                         int head_dim, int block_size, int64_t num_blocks, float scale,
                         int pool_dtype);

/* Same computation carried out in double precision (the reference's golden
 * precedent: crates/core/tests/golden/mod.rs:4-26). */
int orc_decode_attention_f64(double* out, const float* q, const void* k_pool,
                             const void* v_pool, const int32_t* block_tables,
                             int max_blocks_per_seq, const int32_t* ctx_lens, int num_seqs,
                             int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                             int64_t num_blocks, float scale, int pool_dtype);

/* Split-K form.  Pass 1 writes, per (b, h, partition p) of partition_size
 * tokens: m = max_j s_j, l = sum_j e^{s_j-m}, acc[d] = sum_j e^{s_j-m} v_j[d]
 * into m/l [B, Hq, max_parts] and acc [B, Hq, max_parts, D].  Pass 2 merges
 * with the online-softmax rule of ContextParallel::update_online_softmax /
 * finalize_output (crates/distributed/src/context_parallel.rs:300-333):
 *   M = max_p m_p, o = sum_p e^{m_p-M} acc_p / sum_p e^{m_p-M} l_p. */
int orc_decode_partials(float* m, float* l, float* acc, const float* q, const void* k_pool,
                        const void* v_pool, const int32_t* block_tables, int max_blocks_per_seq,
                        const int32_t* ctx_lens, int num_seqs, int num_q_heads, int num_kv_heads,
                        int head_dim, int block_size, int64_t num_blocks, float scale,
                        int pool_dtype, int partition_size, int max_parts);
int orc_splitk_merge(float* out, const float* m, const float* l, const float* acc,
                     const int32_t* ctx_lens, int max_blocks_per_seq, int block_size,
                     int num_seqs, int num_q_heads, int head_dim, int partition_size,
                     int max_parts);

/* ---- 1-byte KV storage (CacheQuantization::Int8 / Fp8) ------------------
 * The reference declares the modes (crates/nn/src/kv_cache.rs:38-63) but its
 * quantize_kv (:266-296) divides by the scale and multiplies by 127 again
 * (off by a factor 127, then clamped) and its dequantize_kv (:299-314) is
 * never called, so this is the build's own specification, per row (the
 * head_dim values of one token of one KV head) with an fp32 scale:
 *   int8: amax = max |x|, s = amax / 127, q = rint(x * (127 / amax)) clamped
 *         to [-127, 127] (amax = 0 or NaN input: 0); value = q * s.
 *   fp8 (OCP e4m3, the Fp8 mode): s = amax / 448, q = e4m3(x * (448 / amax))
 *         rounded to nearest even, |.| >= 448 saturating to 448, NaN kept;
 *         value = f32(q) * s.
 * Rows are stored in pools of bytes with the same layout as the fp32/bf16
 * pools and scales in [num_blocks][num_kv_heads][block_size] fp32. */
uint8_t orc_e4m3_from_f32(float x);
float orc_f32_from_e4m3(uint8_t b);
/* Quantizes one row of n values: bytes into q, the scale into *scale. */
void orc_quantize_row(const float* x, int n, int dtype, uint8_t* q, float* scale);
/* orc_append for 1-byte pools: quantizes each (token, head) row into the
 * pool and its scale into the scale pool. */
int orc_append_q(uint8_t* k_pool, uint8_t* v_pool, float* k_scale, float* v_scale,
                 const float* k_new, const float* v_new, const int64_t* slot_mapping,
                 int64_t n_tokens, int num_kv_heads, int head_dim, int block_size,
                 int64_t num_blocks, int64_t src_tok_stride, int64_t src_head_stride, int dtype);
/* value = dequantized byte * its row's scale, for n_rows rows of head_dim. */
void orc_dequantize_pool(const uint8_t* pool, const float* scales, int64_t n_rows, int head_dim,
                         int dtype, float* out);

/* Causal prefill attention over the paged pool.  Sequence b has n_b =
 * q_start[b+1] - q_start[b] new query tokens (rows q_start[b] .. of q/out,
 * [total, Hq, D] fp32) whose K/V are already in the pool; token i sits at
 * position p = ctx_lens[b] - n_b + i and attends to positions 0 .. p.  This
 * is the per-head recipe of forward_tape_with_mask
 * (crates/nn/src/tape_transformer.rs:87-139) with the additive causal mask of
 * causal_mask_tape (:276-296): -1e9 above the diagonal, which underflows to a
 * zero weight in the softmax, so masked positions drop out exactly.  The
 * reference's square case is ctx_lens[b] == n_b; a larger ctx_lens[b] is a
 * chunked prefill after ctx_lens[b] - n_b cached tokens.  Each row is
 * orc_decode_attention's computation with L = p + 1 (p < 0: zero row). */
int orc_prefill_attention(float* out, const float* q, const void* k_pool, const void* v_pool,
                          const int32_t* block_tables, int max_blocks_per_seq,
                          const int32_t* q_start, const int32_t* ctx_lens, int num_seqs,
                          int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                          int64_t num_blocks, float scale, int pool_dtype);

/* orc_decode_attention split over n_threads POSIX threads by (b, kv head);
 * identical results (each output is computed by one thread in the same
 * order).  Used only as the CPU baseline timing. */
int orc_decode_attention_mt(float* out, const float* q, const void* k_pool, const void* v_pool,
                            const int32_t* block_tables, int max_blocks_per_seq,
                            const int32_t* ctx_lens, int num_seqs, int num_q_heads,
                            int num_kv_heads, int head_dim, int block_size, int64_t num_blocks,
                            float scale, int pool_dtype, int n_threads);

/* ---- config-0 decoder: the model glue around the path ------------------
 * A pre-LN causal decoder with KV-cached single-token steps:
 *   x = E[id] + PE[pos]                  Embedding gather_rows (lib.rs:462-475),
 *                                        sinusoidal PE (transformer.rs:69-82)
 *   per layer:  h = LN1(x); q,k,v = h W^T + b; cache k,v at pos;
 *               a = MHA(q, cache[0..pos]) W_o^T + b_o;  x = x + a
 *               h = LN2(x); x = x + (gelu(h W_1^T + b_1)) W_2^T + b_2
 *                                        (tape_transformer.rs:209-247 block order,
 *                                        :87-139 per-head attention)
 *   logits = LN_f(x) W_lm^T              (lm_head has no bias, transformer.rs:789)
 *   next = argmax(logits)                (orc_argmax)
 * The prompt is fed one token per step (equal to a causal prefill).
 * Parameters are one float array in this order (kvd = n_kv_heads * d_head):
 *   embed[V][d]
 *   per layer: ln1_g[d] ln1_b[d] wq[d][d] bq[d] wk[kvd][d] bk[kvd] wv[kvd][d]
 *              bv[kvd] wo[d][d] bo[d] ln2_g[d] ln2_b[d] w1[f][d] b1[f]
 *              w2[d][f] b2[d]
 *   lnf_g[d] lnf_b[d] lm_head[V][d]
 * Weights are [out][in] as the reference's Linear stores them. */
typedef struct {
  int vocab, d_model, n_heads, n_kv_heads, d_ff, n_layers, max_seq;
  float eps;
} orc_decoder_config;

int64_t orc_decoder_param_count(const orc_decoder_config* c);

/* CpuOps::linear (lib.rs:478-534): y[r][o] = sum_i x[r][i] * w[o][i], summed
 * serially in i without fused multiply-add, then add_row_vector (:318-341)
 * of b (skipped if b is NULL). */
void orc_linear(float* y, const float* x, const float* w, const float* b, int rows, int in_dim,
                int out_dim);

/* LayerNorm::forward (crates/nn/src/normalization.rs:113-157): per row,
 * mean = serial sum / n, var = serial sum of (x-mean)^2 / n,
 * y = (x - mean) / sqrt(var + eps) * g + b. */
void orc_layer_norm(float* y, const float* x, const float* g, const float* b, int rows, int dim,
                    float eps);

/* CpuOps::gelu (lib.rs:565-598), tanh form, element-wise. */
void orc_gelu(float* y, const float* x, int64_t n);

/* PositionalEncoding::new (crates/nn/src/transformer.rs:69-82): pe[pos][i] =
 * sin or cos of pos / 10000^(2*(i/2)/d), in fp32. */
void orc_positional_encoding(float* pe, int max_len, int d_model);

/* Greedy generation: feeds n_prompt prompt ids, then n_new - 1 generated ids,
 * writing the n_new generated ids (and, if out_logits != NULL, the logits
 * [n_new][vocab] each was chosen from).  Returns 0, or -1 on bad args. */
int orc_decoder_generate(const orc_decoder_config* c, const float* params,
                         const int32_t* prompt, int n_prompt, int n_new, int32_t* out_tokens,
                         float* out_logits);

#ifdef __cplusplus
}
#endif
#endif
