/*
 * rustral_model.h -- the model glue around the paged-KV path in
 * librustral_kv.so: the TensorOps subset a decoder step needs on the device,
 * a greedy decoder (benchmark configs[0]) built from them and the paged-KV
 * entry points of rustral_kv.h, and the seeded parameter generator.
 *
 * Conventions are those of rustral_kv.h (device pointers unless marked host,
 * opaque stream, int status + rkv_last_error()).  Every op is fp32 and sums
 * in the order the reference's ndarray backend does (serial sums, no fused
 * multiply-add), so linear, layer_norm, add and argmax give the same bits as
 * that CPU path; gelu uses the device tanhf (within a few ulps of libm).
 */
#ifndef RUSTRAL_MODEL_H
#define RUSTRAL_MODEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- TensorOps subset ----------------------------------------------------- */

/* out[t][i] = table[ids[t]][i] + pe[positions[t]][i].
 * Replaces TensorOps::gather_rows (crates/ndarray-backend/src/lib.rs:462-475)
 * followed by PositionalEncoding's add (crates/nn/src/transformer.rs:64-104).
 * An id outside [0, vocab) or a position outside [0, max_len) gives a row of
 * NaN (the reference returns CoreError::InvalidArgument).  pe may be NULL
 * (no positional term). */
int rkv_embed(float* out, const float* table, const int32_t* ids, const float* pe,
              const int32_t* positions, int n_tokens, int vocab, int dim, int max_len,
              void* stream);

/* y[r][o] = sum_i x[r][i] * w[o][i] + b[o], the sum serial in i.
 * Replaces TensorOps::linear (lib.rs:478-534) + add_row_vector (:318-341).
 * w is [out_dim][in_dim] (the reference's Linear layout); b may be NULL;
 * in_dim <= 8192. */
int rkv_linear(float* y, const float* x, const float* w, const float* b, int rows, int in_dim,
               int out_dim, void* stream);

/* Per row: mean and biased variance by serial sums, then
 * (x - mean) / sqrt(var + eps) * g + b.  Replaces LayerNorm::forward
 * (crates/nn/src/normalization.rs:113-157).  dim <= 8192. */
int rkv_layer_norm(float* y, const float* x, const float* g, const float* b, int rows, int dim,
                   float eps, void* stream);

/* The attention input of one decoder layer in one launch, for n_tokens rows
 * of x [n_tokens][d_model]:
 *   h = LayerNorm(x; ln_g, ln_b, eps)   (ln_g == ln_b == NULL: h = x)
 *   q_out[t] = h[t] wq^T + bq           ([n_tokens][q_dim], wq [q_dim][d_model])
 *   k = h wk^T + bk, v = h wv^T + bv    (wk, wv [num_kv_heads*head_dim][d_model])
 * and k[t], v[t] appended to the paged pools at slot_mapping[t] as rkv_append
 * does (pool layout [num_blocks][num_kv_heads][block_size][head_dim], dtype
 * RKV_F32 or RKV_BF16; a slot outside the pool appends nothing).  Biases may
 * be NULL.  The arithmetic and its order are those of rkv_layer_norm, three
 * rkv_linear calls and rkv_append, so the results are the same bits.
 * Replaces the pre-norm and q / k / v projections of the reference's layer
 * (crates/nn/src/tape_transformer.rs:242 ln1, :94-96 wq / wk / wv) followed by
 * the KV append (KVCache::append, crates/nn/src/kv_cache.rs:172-216).
 * d_model <= 8192, n_tokens <= 65535. */
int rkv_qkv_append(float* q_out, void* k_pool, void* v_pool, const int64_t* slot_mapping,
                   const float* x, const float* ln_g, const float* ln_b, float eps,
                   const float* wq, const float* bq, const float* wk, const float* bk,
                   const float* wv, const float* bv, int n_tokens, int d_model, int q_dim,
                   int num_kv_heads, int head_dim, int block_size, int64_t num_blocks,
                   int dtype, void* stream);

/* 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).  Replaces TensorOps::gelu
 * (lib.rs:565-598). */
int rkv_gelu(float* y, const float* x, int64_t n, void* stream);

/* y = a + b element-wise.  Replaces TensorOps::add (lib.rs:283-315). */
int rkv_add(float* y, const float* a, const float* b, int64_t n, void* stream);

/* y = x * s element-wise.  Replaces TensorOps::mul_scalar (lib.rs:747-756). */
int rkv_mul_scalar(float* y, const float* x, float s, int64_t n, void* stream);

/* Softmax along one axis of a tensor viewed as [outer][axis][inner]: per
 * line, max (NaN skipped, as f32::max), e = exp(x - max), sum = the e added
 * serially in axis order, y = e * (1 / sum).  Replaces TensorOps::softmax_dim
 * (crates/ndarray-backend/src/lib.rs:1188-1227; dim d of shape s gives
 * outer = prod s[..d], axis = s[d], inner = prod s[d+1..]).  axis == 0 is
 * RKV_ERR_INVALID_ARG, the reference's "axis size is 0".  exp is the device
 * library's expf (within 2 ulp of the host's). */
int rkv_softmax_dim(float* y, const float* x, int64_t outer, int64_t axis, int64_t inner,
                    void* stream);

/* y[m][n] = sum_j a[m][j] * b[j][n] (row-major), each sum serial in j without
 * fused multiply-add: the order of TensorOps::matmul's naive loop
 * (lib.rs:191-267; the reference hands products with m*k*n >= 64 to the
 * matrixmultiply crate's sgemm, whose blocked order is not reproduced).
 * m <= 1048560. */
int rkv_matmul(float* y, const float* a, const float* b, int m, int k, int n, void* stream);

/* y[n][m] = x[m][n] (y must not alias x).  Replaces TensorOps::transpose
 * (lib.rs:270-281).  m <= 2097120. */
int rkv_transpose(float* y, const float* x, int m, int n, void* stream);

/* out[r] = index of the maximum of row r (n columns), the LAST one among
 * equal maxima; NaN compares equal to everything, as in TensorOps::argmax
 * (lib.rs:430-437) and Sampler::greedy (crates/nn/src/continuous_batching.rs:
 * 458-462), i.e. the result is that of a left-to-right scan that moves to
 * element i unless the current best is greater. */
int rkv_argmax(int32_t* out, const float* x, int rows, int n, void* stream);

/* ---- greedy decoder (benchmark configs[0]) ------------------------------------
 * Pre-LN causal decoder: x = E[id] + PE[pos]; per layer h = LN1(x),
 * q,k,v = h W^T + b, K/V appended to a paged fp32 pool (16-token blocks from
 * a host block manager), a = paged decode attention (rkv_decode_attention)
 * W_o^T + b_o, x += a, x += W_2 gelu(W_1 LN2(x) + b_1) + b_2; logits =
 * LN_f(x) W_lm^T; next id = argmax.  The prompt is fed one token per step
 * (equal to a causal prefill: each step attends to the cache including
 * itself).  Follows tape_transformer.rs:87-139 (per-head attention) and
 * :209-247 (pre-LN block), transformer.rs:69-82 (PE) and :789 (lm_head
 * without bias).
 *
 * Parameters: one fp32 host array, in this order (kvd = n_kv_heads*d_head):
 *   embed[V][d]
 *   per layer: ln1_g[d] ln1_b[d] wq[d][d] bq[d] wk[kvd][d] bk[kvd] wv[kvd][d]
 *              bv[kvd] wo[d][d] bo[d] ln2_g[d] ln2_b[d] w1[f][d] b1[f]
 *              w2[d][f] b2[d]
 *   lnf_g[d] lnf_b[d] lm_head[V][d]                                          */
typedef struct {
  int vocab, d_model, n_heads, n_kv_heads, d_ff, n_layers, max_seq;
  float eps;
} rkv_decoder_config;

typedef struct rkv_decoder rkv_decoder;

/* Floats in the parameter array of a configuration (-1 if invalid). */
int64_t rkv_decoder_param_count(const rkv_decoder_config* cfg);

/* Random initialisation (host): every weight matrix and the embedding
 * N(0, std^2) from one rkv_fill_normal stream (seed) in parameter order;
 * layer-norm gains 1, biases and betas 0.  The reference's normal_parameter
 * draws U[-scale, scale) from rand's StdRng (crates/ndarray-backend/src/
 * lib.rs:132-146), which this build does not reproduce. */
int rkv_decoder_init_params(const rkv_decoder_config* cfg, uint64_t seed, float std,
                            float* host_params);

/* Uploads host_params (rkv_decoder_param_count floats) and allocates the
 * paged KV pools (ceil(max_seq / 16) blocks per layer) on the current
 * device.  stream NULL: the decoder creates a stream of its own.  NULL on
 * failure (rkv_last_error).  Supported: d_model / n_heads in {32, 64, 128},
 * n_heads / n_kv_heads in {1, 2, 4, 8}. */
rkv_decoder* rkv_decoder_create(const rkv_decoder_config* cfg, const float* host_params,
                                int64_t n_params, void* stream);
void rkv_decoder_destroy(rkv_decoder* dec);

/* Greedy generation of n_new tokens after n_prompt prompt ids (host arrays).
 * out_tokens: host [n_new]; out_logits: host [n_new][vocab] or NULL.
 * n_prompt + n_new - 1 <= max_seq.  Synchronizes the stream at the end.  The
 * launch sequence of a (n_prompt, n_new) shape is captured into a HIP graph
 * by the first call of that shape and replayed by later ones. */
int rkv_decoder_generate(rkv_decoder* dec, const int32_t* prompt, int n_prompt, int n_new,
                         int32_t* out_tokens, float* out_logits);

/* ---- parameters in safetensors files (host) ---------------------------------------
 * The reference saves and loads models as safetensors keyed by stable
 * parameter names (crates/runtime/src/model_io.rs:12-33 save_model, :36-105
 * load_model: strict -- missing keys, extra keys, a shape or element-count
 * mismatch and a dtype other than F32 are errors; __metadata__ is ignored).
 * Names, in parameter order (kvd = n_kv_heads * d_head):
 *   token_embedding.weight [V, d]
 *   layers.{i}.norm1.weight / .bias [d]
 *   layers.{i}.self_attn.{q,out}_proj.weight [d, d], .bias [d]
 *   layers.{i}.self_attn.{k,v}_proj.weight [kvd, d], .bias [kvd]
 *   layers.{i}.norm2.weight / .bias [d]
 *   layers.{i}.ff_linear1.weight [f, d], .bias [f]
 *   layers.{i}.ff_linear2.weight [d, f], .bias [d]
 *   final_norm.weight / .bias [d]
 *   lm_head.weight [V, d]
 * (the reference's TransformerDecoder names, transformer.rs:894-935, with a
 * .weight/.bias pair for this decoder's biased projections). */
int rkv_decoder_load_safetensors(const rkv_decoder_config* cfg, const char* path,
                                 float* host_params, int64_t n_params);
int rkv_decoder_save_safetensors(const rkv_decoder_config* cfg, const float* host_params,
                                 int64_t n_params, const char* path);

/* The same strict load straight into a decoder's device parameters (one
 * host-to-device copy per tensor from the memory-mapped file, on the
 * decoder's stream; returns once they are done).  On an error the decoder's
 * parameters are unchanged unless the failure is a HIP copy error. */
int rkv_decoder_load_safetensors_device(rkv_decoder* dec, const char* path);

/* rkv_decoder_create with the parameters read from a safetensors file
 * straight into device memory (no host parameter array).  NULL on failure
 * (rkv_last_error carries load_model's message). */
rkv_decoder* rkv_decoder_create_from_safetensors(const rkv_decoder_config* cfg,
                                                 const char* path, void* stream);

/* ---- any named-parameter model in a safetensors file --------------------------
 * The reference's load_model (crates/runtime/src/model_io.rs:36-105) loads
 * every NamedParameters model the same way; these calls give a caller (the
 * Rust backend, a Llama layer's projections) that load for its own list of
 * names, shapes and destinations.  rkv_st_open maps the file read-only and
 * checks its header (JSON object; every entry with a dtype string, integer
 * shape, data_offsets inside the data section and matching the element count
 * for the known dtypes); NULL on failure. */
typedef struct rkv_st_file rkv_st_file;
rkv_st_file* rkv_st_open(const char* path);
void rkv_st_close(rkv_st_file* f);
int64_t rkv_st_num_tensors(const rkv_st_file* f);
/* Entry i in header order: name and dtype strings (valid until rkv_st_close),
 * number of dimensions, and up to max_dims sizes. */
int rkv_st_tensor(const rkv_st_file* f, int64_t i, const char** name, const char** dtype,
                  int* ndim, int64_t* shape, int max_dims);
/* load_model's strict load: n tensors names[i] with ndims[i] dimensions
 * (shapes concatenated in order), each F32, copied into dsts[i] -- device
 * pointers when dst_on_device (hipMemcpyAsync on stream, finished before the
 * call returns), else host pointers.  Missing keys, keys of the file not in
 * the list, a shape mismatch or another dtype are RKV_ERR_INVALID_ARG with
 * the reference's message. */
int rkv_st_load(const rkv_st_file* f, int n, const char* const* names, const int* ndims,
                const int64_t* shapes, void* const* dsts, int dst_on_device, void* stream);

/* ---- serving engine (continuous batching over the decoder) ----------------------
 * Replaces ServingEngine (crates/nn/src/continuous_batching.rs:493-537).  The
 * reference's step emits a dummy token for every scheduled request
 * (:516-524); here a step runs the decoder above over the scheduler's batch
 * (include/rustral_serving.h, which owns the block manager): all input tokens
 * of the batch as rows -- a prompt in prefill, the last generated token
 * otherwise, prompt + generated when resuming after a preemption -- their K/V
 * appended into paged fp32 pools of num_blocks 16-token blocks per layer, one
 * rkv_prefill_attention call per layer for the whole batch (a decode row is
 * its single-token case), and one greedy token per request from its last
 * row, handed to rkv_sched_update.  Every call synchronizes the stream once
 * (the tokens come back to the host for the scheduler). */
typedef struct rkv_engine rkv_engine;
struct rkv_scheduler;

/* Uploads the parameters and allocates the pools on the current device; the
 * engine's scheduler admits at most max_batch_size running requests and
 * bounds prompt + max_tokens by cfg->max_seq.  NULL on failure. */
rkv_engine* rkv_engine_create(const rkv_decoder_config* cfg, const float* host_params,
                              int64_t n_params, int64_t num_blocks, int max_batch_size,
                              void* stream);
void rkv_engine_destroy(rkv_engine* e);

/* ServingEngine::submit (:507-510): queues a request, returns its id. */
int64_t rkv_engine_submit(rkv_engine* e, const int32_t* prompt, int n_prompt, int max_tokens,
                          int priority);

/* ServingEngine::step (:513-535): returns the number of requests run (0 when
 * nothing is running) or a negative code (RKV_ERR_OOM when the pool cannot
 * hold a request's next token, as Scheduler::update reports it). */
int rkv_engine_step(rkv_engine* e);

/* ServingEngine::run_to_completion (:538-543), bounded by max_steps; returns
 * the number of steps run or a negative code. */
int rkv_engine_run(rkv_engine* e, int max_steps);

/* The engine's scheduler: rkv_sched_generated / rkv_sched_stats read the
 * results.  Owned by the engine. */
struct rkv_scheduler* rkv_engine_scheduler(rkv_engine* e);

/* ---- seeded generator (host) -------------------------------------------------
 * PCG64 (XSL-RR 128/64; state' = state * 0x2360ED051FC65DA44385DF649FCCF645
 * + inc, output from state') with state = seed and inc = 0xDA3E39CB94B95BDB *
 * 2 + 1, the stream numpy's PCG64 gives with that state; uniforms
 * u = (x >> 11) * 2^-53; normals by Box-Muller in double,
 * sqrt(-2 ln(1 - u1)) * (cos, sin)(2 pi u2), both used, rounded to fp32
 * after scaling by std. */
int rkv_rng_raw(uint64_t seed, uint64_t* out, int64_t n);
int rkv_fill_normal(float* out, int64_t n, uint64_t seed, float std);

#ifdef __cplusplus
}
#endif
#endif /* RUSTRAL_MODEL_H */
