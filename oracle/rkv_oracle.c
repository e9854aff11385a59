/*
 * rkv_oracle.c -- CPU restatement of rustral's paged-KV hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see rkv_oracle.h): the checker for the HIP
 * library, never part of the product path.
 *
 * Built with -O2 -ffp-contract=off so every float operation is rounded in
 * program order, like the reference's scalar Rust loops.
 */
#include "rkv_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---- bf16 -------------------------------------------------------------- */

uint16_t orc_bf16_from_f32(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) /* NaN: keep sign/payload, set quiet bit */
    return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u); /* round to nearest, ties to even */
  return (uint16_t)(u >> 16);
}

float orc_f32_from_bf16(uint16_t b) {
  uint32_t u = (uint32_t)b << 16; /* as bf16_to_f32, compression.rs:263-267 */
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void orc_bf16_from_f32_array(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_bf16_from_f32(x[i]);
}

void orc_f32_from_bf16_array(const uint16_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_from_bf16(x[i]);
}

static inline float load_elem(const void* pool, int dtype, int64_t idx) {
  if (dtype == ORC_F32) return ((const float*)pool)[idx];
  return orc_f32_from_bf16(((const uint16_t*)pool)[idx]);
}

static inline size_t dtype_size(int dtype) { return dtype == ORC_F32 ? 4 : 2; }

/* ---- append ------------------------------------------------------------ */

int orc_append(void* k_pool, void* v_pool, const float* k_new, const float* v_new,
               const int64_t* slot_mapping, int64_t n_tokens, int num_kv_heads, int head_dim,
               int block_size, int64_t num_blocks, int64_t src_tok_stride,
               int64_t src_head_stride, int pool_dtype) {
  if (!k_pool || !v_pool || !k_new || !v_new || !slot_mapping) return -1;
  if (n_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0) return -1;
  if (pool_dtype != ORC_F32 && pool_dtype != ORC_BF16) return -1;
  const int64_t n_slots = num_blocks * block_size;
  for (int64_t t = 0; t < n_tokens; ++t) {
    const int64_t slot = slot_mapping[t];
    if (slot < 0 || slot >= n_slots) continue;
    const int64_t blk = slot / block_size, row = slot % block_size;
    for (int h = 0; h < num_kv_heads; ++h) {
      const int64_t dst = ((blk * num_kv_heads + h) * block_size + row) * head_dim;
      const int64_t src = t * src_tok_stride + (int64_t)h * src_head_stride;
      for (int d = 0; d < head_dim; ++d) {
        if (pool_dtype == ORC_F32) {
          ((float*)k_pool)[dst + d] = k_new[src + d];
          ((float*)v_pool)[dst + d] = v_new[src + d];
        } else {
          ((uint16_t*)k_pool)[dst + d] = orc_bf16_from_f32(k_new[src + d]);
          ((uint16_t*)v_pool)[dst + d] = orc_bf16_from_f32(v_new[src + d]);
        }
      }
    }
  }
  return 0;
}

/* ---- 1-byte storage ------------------------------------------------------ */

uint8_t orc_e4m3_from_f32(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  const uint32_t sign = (u >> 24) & 0x80u, a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7fu); /* NaN */
  if (a >= 0x43e00000u) return (uint8_t)(sign | 0x7eu); /* >= 448 saturates */
  if (a < 0x3c800000u) { /* below 2^-6: subnormal m * 2^-9 */
    float f;
    memcpy(&f, &a, 4);
    return (uint8_t)(sign | (uint32_t)(int)rintf(f * 512.0f));
  }
  uint32_t e = (a >> 23) - 120u, m = (a >> 20) & 7u;
  const uint32_t rem = a & 0xfffffu;
  if (rem > 0x80000u || (rem == 0x80000u && (m & 1u))) ++m; /* nearest, ties to even */
  if (m == 8u) {
    m = 0;
    ++e;
  }
  return (uint8_t)(sign | (e << 3) | m);
}

float orc_f32_from_e4m3(uint8_t b) {
  const int e = (b >> 3) & 15, m = b & 7;
  float v;
  if (e == 15 && m == 7)
    v = NAN;
  else if (e == 0)
    v = (float)m * 0.001953125f; /* m * 2^-9 */
  else
    v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return (b & 0x80) ? -v : v;
}

static uint8_t i8_quant(float x, float inv) {
  const float r = rintf(x * inv);
  if (r != r) return 0;
  const float c = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
  return (uint8_t)(int8_t)(int)c;
}

void orc_quantize_row(const float* x, int n, int dtype, uint8_t* q, float* scale) {
  float amax = 0.0f;
  for (int i = 0; i < n; ++i) amax = fmaxf(amax, fabsf(x[i]));
  const float top = dtype == ORC_I8 ? 127.0f : 448.0f;
  const float inv = amax > 0.0f ? top / amax : 0.0f;
  *scale = amax / top;
  for (int i = 0; i < n; ++i)
    q[i] = dtype == ORC_I8 ? i8_quant(x[i], inv) : orc_e4m3_from_f32(x[i] * inv);
}

int orc_append_q(uint8_t* k_pool, uint8_t* v_pool, float* k_scale, float* v_scale,
                 const float* k_new, const float* v_new, const int64_t* slot_mapping,
                 int64_t n_tokens, int num_kv_heads, int head_dim, int block_size,
                 int64_t num_blocks, int64_t src_tok_stride, int64_t src_head_stride, int dtype) {
  if (!k_pool || !v_pool || !k_scale || !v_scale || !k_new || !v_new || !slot_mapping) return -1;
  if (dtype != ORC_I8 && dtype != ORC_FP8) return -1;
  const int64_t n_slots = num_blocks * block_size;
  for (int64_t t = 0; t < n_tokens; ++t) {
    const int64_t slot = slot_mapping[t];
    if (slot < 0 || slot >= n_slots) continue;
    const int64_t blk = slot / block_size, row = slot % block_size;
    for (int h = 0; h < num_kv_heads; ++h) {
      const int64_t r = (blk * num_kv_heads + h) * block_size + row;
      const int64_t src = t * src_tok_stride + (int64_t)h * src_head_stride;
      orc_quantize_row(k_new + src, head_dim, dtype, k_pool + r * head_dim, k_scale + r);
      orc_quantize_row(v_new + src, head_dim, dtype, v_pool + r * head_dim, v_scale + r);
    }
  }
  return 0;
}

void orc_dequantize_pool(const uint8_t* pool, const float* scales, int64_t n_rows, int head_dim,
                         int dtype, float* out) {
  for (int64_t r = 0; r < n_rows; ++r)
    for (int d = 0; d < head_dim; ++d) {
      const uint8_t b = pool[r * head_dim + d];
      const float v = dtype == ORC_I8 ? (float)(int8_t)b : orc_f32_from_e4m3(b);
      out[r * head_dim + d] = v * scales[r];
    }
}

/* ---- gather ------------------------------------------------------------ */

static inline int clamp_ctx(int L, int max_blocks_per_seq, int block_size) {
  const int cap = max_blocks_per_seq * block_size;
  if (L < 0) return 0;
  return L > cap ? cap : L;
}

int orc_gather(void* k_out, void* v_out, const void* k_pool, const void* v_pool,
               const int32_t* block_tables, int max_blocks_per_seq, const int32_t* ctx_lens,
               const int64_t* out_offsets, int num_seqs, int num_kv_heads, int head_dim,
               int block_size, int64_t num_blocks, int max_ctx, int pool_dtype, int out_dtype) {
  if (!k_out || !v_out || !k_pool || !v_pool || !block_tables || !ctx_lens) return -1;
  if (out_dtype != ORC_F32 && out_dtype != pool_dtype) return -1;
  for (int b = 0; b < num_seqs; ++b) {
    const int L = clamp_ctx(ctx_lens[b], max_blocks_per_seq, block_size);
    if (!out_offsets && L > max_ctx) return -1;
    for (int p = 0; p < L; ++p) {
      const int32_t blk = block_tables[(int64_t)b * max_blocks_per_seq + p / block_size];
      if (blk < 0 || blk >= num_blocks) continue;
      const int row = p % block_size;
      for (int h = 0; h < num_kv_heads; ++h) {
        const int64_t src = (((int64_t)blk * num_kv_heads + h) * block_size + row) * head_dim;
        int64_t dst;
        if (out_offsets)
          dst = out_offsets[b] + ((int64_t)h * L + p) * head_dim;
        else
          dst = (((int64_t)b * num_kv_heads + h) * max_ctx + p) * head_dim;
        if (out_dtype == pool_dtype) {
          const size_t es = dtype_size(pool_dtype);
          memcpy((char*)k_out + dst * es, (const char*)k_pool + src * es, head_dim * es);
          memcpy((char*)v_out + dst * es, (const char*)v_pool + src * es, head_dim * es);
        } else {
          for (int d = 0; d < head_dim; ++d) {
            ((float*)k_out)[dst + d] = load_elem(k_pool, pool_dtype, src + d);
            ((float*)v_out)[dst + d] = load_elem(v_pool, pool_dtype, src + d);
          }
        }
      }
    }
  }
  return 0;
}

/* ---- copy_blocks ------------------------------------------------------- */

int orc_copy_blocks(void* k_pool, void* v_pool, int64_t layer_stride_bytes, int n_layers,
                    const int32_t* pairs, int n_pairs, int64_t block_bytes, int64_t num_blocks) {
  if (!k_pool || !v_pool || (n_pairs > 0 && !pairs) || block_bytes <= 0) return -1;
  for (int l = 0; l < n_layers; ++l) {
    char* kp = (char*)k_pool + (int64_t)l * layer_stride_bytes;
    char* vp = (char*)v_pool + (int64_t)l * layer_stride_bytes;
    for (int i = 0; i < n_pairs; ++i) {
      const int32_t src = pairs[2 * i], dst = pairs[2 * i + 1];
      if (src < 0 || src >= num_blocks || dst < 0 || dst >= num_blocks) continue;
      memmove(kp + (int64_t)dst * block_bytes, kp + (int64_t)src * block_bytes, block_bytes);
      memmove(vp + (int64_t)dst * block_bytes, vp + (int64_t)src * block_bytes, block_bytes);
    }
  }
  return 0;
}

/* ---- softmax / argmax -------------------------------------------------- */

/* CpuOps::softmax_dim (crates/ndarray-backend/src/lib.rs:1188-1227): the
 * loops over (o, i), each line's max from -inf by f32::max (fmaxf: a NaN
 * operand is skipped), exp, serial sum and the 1/sum scale, in that order. */
int orc_softmax_dim(const float* x, float* y, int64_t outer, int64_t axis, int64_t inner) {
  if (axis <= 0 || outer < 0 || inner < 0) return -1; /* lib.rs:1200-1202 */
  for (int64_t o = 0; o < outer; ++o) {
    for (int64_t i = 0; i < inner; ++i) {
      const int64_t base = o * axis * inner + i;
      float mx = -INFINITY;
      for (int64_t a = 0; a < axis; ++a) mx = fmaxf(mx, x[base + a * inner]);
      float sum = 0.0f;
      for (int64_t a = 0; a < axis; ++a) {
        const float e = expf(x[base + a * inner] - mx);
        y[base + a * inner] = e;
        sum += e;
      }
      const float inv = 1.0f / sum;
      for (int64_t a = 0; a < axis; ++a) y[base + a * inner] *= inv;
    }
  }
  return 0;
}

void orc_softmax_rows(const float* x, float* y, int rows, int cols) {
  orc_softmax_dim(x, y, rows, cols, 1);
}

/* CpuOps::matmul's naive loop (lib.rs:208-219): out[i][j] = sum over kk of
 * a[i][kk] * b[kk][j], serial in kk from 0.0. */
void orc_matmul(const float* a, const float* b, float* y, int m, int k, int n) {
  for (int i = 0; i < m; ++i)
    for (int j = 0; j < n; ++j) {
      float sum = 0.0f;
      for (int kk = 0; kk < k; ++kk) sum += a[(int64_t)i * k + kk] * b[(int64_t)kk * n + j];
      y[(int64_t)i * n + j] = sum;
    }
}

/* CpuOps::transpose (lib.rs:270-281): out[j][i] = x[i][j]. */
void orc_transpose(const float* x, float* y, int m, int n) {
  for (int i = 0; i < m; ++i)
    for (int j = 0; j < n; ++j) y[(int64_t)j * m + i] = x[(int64_t)i * n + j];
}

/* CpuOps::mul_scalar (lib.rs:747-756): v * scalar per element. */
void orc_mul_scalar(const float* x, float* y, float s, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = x[i] * s;
}

int64_t orc_argmax(const float* x, int64_t n) {
  if (n <= 0) return -1;
  /* max_by keeps the later element when the comparison says Equal; NaN
   * compares Equal through unwrap_or(Equal) (ndarray-backend/src/lib.rs:434). */
  int64_t best = 0;
  for (int64_t i = 1; i < n; ++i) {
    const float a = x[best], b = x[i];
    const int less = a < b, greater = a > b;
    if (less || (!less && !greater)) best = i; /* b >= a, or unordered */
  }
  return best;
}

/* ---- decode attention -------------------------------------------------- */

typedef struct {
  const float* q;
  const void* k_pool;
  const void* v_pool;
  const int32_t* block_tables;
  const int32_t* ctx_lens;
  int max_blocks_per_seq, num_q_heads, num_kv_heads, head_dim, block_size, pool_dtype;
  int64_t num_blocks;
  float scale;
} dec_args;

static int check_dec(const float* q, const void* k, const void* v, const int32_t* bt,
                     const int32_t* cl, int nq, int nkv, int d, int bs) {
  if (!q || !k || !v || !bt || !cl) return -1;
  if (nq <= 0 || nkv <= 0 || d <= 0 || bs <= 0 || nq % nkv) return -1;
  return 0;
}

/* Row index of token j in the pool for KV head kh, or -1 if its block id is
 * invalid. */
static inline int64_t token_row(const dec_args* a, int b, int kh, int j) {
  const int32_t blk = a->block_tables[(int64_t)b * a->max_blocks_per_seq + j / a->block_size];
  if (blk < 0 || blk >= a->num_blocks) return -1;
  return (((int64_t)blk * a->num_kv_heads + kh) * a->block_size + j % a->block_size) *
         a->head_dim;
}

/* One (b, h) row in fp32, ndarray op order.  scratch holds L floats. */
static void decode_one_f32(const dec_args* a, int b, int h, float* out, float* s) {
  const int D = a->head_dim;
  const int kh = h / (a->num_q_heads / a->num_kv_heads);
  const int L = clamp_ctx(a->ctx_lens[b], a->max_blocks_per_seq, a->block_size);
  const float* qv = a->q + ((int64_t)b * a->num_q_heads + h) * D;
  for (int d = 0; d < D; ++d) out[d] = 0.0f;
  if (L == 0) return;
  float mx = -INFINITY;
  for (int j = 0; j < L; ++j) {
    const int64_t r = token_row(a, b, kh, j);
    if (r < 0) {
      s[j] = -INFINITY;
      continue;
    }
    float dot = 0.0f; /* matmul: sum += a*b over kk (lib.rs:211-214) */
    for (int d = 0; d < D; ++d) dot += qv[d] * load_elem(a->k_pool, a->pool_dtype, r + d);
    s[j] = dot * a->scale; /* mul_scalar (lib.rs:747-756) */
    mx = fmaxf(mx, s[j]);
  }
  if (mx == -INFINITY) return; /* every block id invalid */
  float sum = 0.0f;
  for (int j = 0; j < L; ++j) {
    const float e = (s[j] == -INFINITY) ? 0.0f : expf(s[j] - mx);
    s[j] = e;
    sum += e;
  }
  const float inv = 1.0f / sum;
  for (int j = 0; j < L; ++j) s[j] *= inv;
  /* weights[1,L] @ vh[L,D]: out[d] = sum over j in order (lib.rs:211-214) */
  for (int j = 0; j < L; ++j) {
    const int64_t r = token_row(a, b, kh, j);
    if (r < 0) continue;
    for (int d = 0; d < D; ++d) out[d] += s[j] * load_elem(a->v_pool, a->pool_dtype, r + d);
  }
}

static int max_ctx_of(const int32_t* cl, int B, int mbs, int bs) {
  int m = 1;
  for (int b = 0; b < B; ++b) {
    const int L = clamp_ctx(cl[b], mbs, bs);
    if (L > m) m = L;
  }
  return m;
}

int orc_decode_attention(float* out, const float* q, const void* k_pool, const void* v_pool,
                         const int32_t* block_tables, int max_blocks_per_seq,
                         const int32_t* ctx_lens, int num_seqs, int num_q_heads, int num_kv_heads,
                         int head_dim, int block_size, int64_t num_blocks, float scale,
                         int pool_dtype) {
  if (!out || check_dec(q, k_pool, v_pool, block_tables, ctx_lens, num_q_heads, num_kv_heads,
                        head_dim, block_size))
    return -1;
  dec_args a = {q, k_pool, v_pool, block_tables, ctx_lens, max_blocks_per_seq, num_q_heads,
                num_kv_heads, head_dim, block_size, pool_dtype, num_blocks, scale};
  float* s = (float*)malloc(sizeof(float) * max_ctx_of(ctx_lens, num_seqs, max_blocks_per_seq,
                                                       block_size));
  if (!s) return -1;
  for (int b = 0; b < num_seqs; ++b)
    for (int h = 0; h < num_q_heads; ++h)
      decode_one_f32(&a, b, h, out + ((int64_t)b * num_q_heads + h) * head_dim, s);
  free(s);
  return 0;
}

int orc_prefill_attention(float* out, const float* q, const void* k_pool, const void* v_pool,
                          const int32_t* block_tables, int max_blocks_per_seq,
                          const int32_t* q_start, const int32_t* ctx_lens, int num_seqs,
                          int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                          int64_t num_blocks, float scale, int pool_dtype) {
  if (!out || !q_start ||
      check_dec(q, k_pool, v_pool, block_tables, ctx_lens, num_q_heads, num_kv_heads, head_dim,
                block_size))
    return -1;
  const int cap = max_blocks_per_seq * block_size;
  float* s = (float*)malloc(sizeof(float) * (cap > 0 ? cap : 1));
  if (!s) return -1;
  for (int b = 0; b < num_seqs; ++b) {
    const int n = q_start[b + 1] - q_start[b];
    for (int i = 0; i < n; ++i) {
      const int64_t row = (int64_t)q_start[b] + i;
      const int p = ctx_lens[b] - n + i;
      int L = p + 1; /* the token attends to positions 0 .. p (causal) */
      /* one decode row: sequence b's table, context L, this token's queries */
      dec_args a = {q + row * num_q_heads * head_dim, k_pool, v_pool,
                    block_tables + (int64_t)b * max_blocks_per_seq, &L, max_blocks_per_seq,
                    num_q_heads, num_kv_heads, head_dim, block_size, pool_dtype, num_blocks, scale};
      for (int h = 0; h < num_q_heads; ++h)
        decode_one_f32(&a, 0, h, out + (row * num_q_heads + h) * head_dim, s);
    }
  }
  free(s);
  return 0;
}

int orc_decode_attention_f64(double* out, const float* q, const void* k_pool,
                             const void* v_pool, const int32_t* block_tables,
                             int max_blocks_per_seq, const int32_t* ctx_lens, int num_seqs,
                             int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                             int64_t num_blocks, float scale, int pool_dtype) {
  if (!out || check_dec(q, k_pool, v_pool, block_tables, ctx_lens, num_q_heads, num_kv_heads,
                        head_dim, block_size))
    return -1;
  dec_args a = {q, k_pool, v_pool, block_tables, ctx_lens, max_blocks_per_seq, num_q_heads,
                num_kv_heads, head_dim, block_size, pool_dtype, num_blocks, scale};
  double* s = (double*)malloc(sizeof(double) * max_ctx_of(ctx_lens, num_seqs,
                                                          max_blocks_per_seq, block_size));
  if (!s) return -1;
  const int G = num_q_heads / num_kv_heads, D = head_dim;
  for (int b = 0; b < num_seqs; ++b) {
    const int L = clamp_ctx(ctx_lens[b], max_blocks_per_seq, block_size);
    for (int h = 0; h < num_q_heads; ++h) {
      double* o = out + ((int64_t)b * num_q_heads + h) * D;
      const float* qv = q + ((int64_t)b * num_q_heads + h) * D;
      for (int d = 0; d < D; ++d) o[d] = 0.0;
      double mx = -INFINITY;
      for (int j = 0; j < L; ++j) {
        const int64_t r = token_row(&a, b, h / G, j);
        if (r < 0) {
          s[j] = -INFINITY;
          continue;
        }
        double dot = 0.0;
        for (int d = 0; d < D; ++d)
          dot += (double)qv[d] * (double)load_elem(k_pool, pool_dtype, r + d);
        s[j] = dot * (double)scale;
        if (s[j] > mx) mx = s[j];
      }
      if (L == 0 || mx == -INFINITY) continue;
      double sum = 0.0;
      for (int j = 0; j < L; ++j) {
        s[j] = (s[j] == -INFINITY) ? 0.0 : exp(s[j] - mx);
        sum += s[j];
      }
      for (int j = 0; j < L; ++j) {
        const int64_t r = token_row(&a, b, h / G, j);
        if (r < 0) continue;
        const double p = s[j] / sum;
        for (int d = 0; d < D; ++d) o[d] += p * (double)load_elem(v_pool, pool_dtype, r + d);
      }
    }
  }
  free(s);
  return 0;
}

/* ---- split-K ----------------------------------------------------------- */

int orc_decode_partials(float* m, float* l, float* acc, const float* q, const void* k_pool,
                        const void* v_pool, const int32_t* block_tables, int max_blocks_per_seq,
                        const int32_t* ctx_lens, int num_seqs, int num_q_heads, int num_kv_heads,
                        int head_dim, int block_size, int64_t num_blocks, float scale,
                        int pool_dtype, int partition_size, int max_parts) {
  if (!m || !l || !acc || partition_size <= 0 ||
      check_dec(q, k_pool, v_pool, block_tables, ctx_lens, num_q_heads, num_kv_heads, head_dim,
                block_size))
    return -1;
  dec_args a = {q, k_pool, v_pool, block_tables, ctx_lens, max_blocks_per_seq, num_q_heads,
                num_kv_heads, head_dim, block_size, pool_dtype, num_blocks, scale};
  const int G = num_q_heads / num_kv_heads, D = head_dim;
  float* s = (float*)malloc(sizeof(float) * partition_size);
  if (!s) return -1;
  for (int b = 0; b < num_seqs; ++b) {
    const int L = clamp_ctx(ctx_lens[b], max_blocks_per_seq, block_size);
    const int np = (L + partition_size - 1) / partition_size;
    if (np > max_parts) {
      free(s);
      return -1;
    }
    for (int h = 0; h < num_q_heads; ++h) {
      const float* qv = q + ((int64_t)b * num_q_heads + h) * D;
      for (int p = 0; p < np; ++p) {
        const int64_t o = ((int64_t)b * num_q_heads + h) * max_parts + p;
        const int j0 = p * partition_size;
        const int j1 = (j0 + partition_size < L) ? j0 + partition_size : L;
        float mx = -INFINITY;
        for (int j = j0; j < j1; ++j) {
          const int64_t r = token_row(&a, b, h / G, j);
          float v = -INFINITY;
          if (r >= 0) {
            float dot = 0.0f;
            for (int d = 0; d < D; ++d) dot += qv[d] * load_elem(k_pool, pool_dtype, r + d);
            v = dot * scale;
          }
          s[j - j0] = v;
          mx = fmaxf(mx, v);
        }
        float sum = 0.0f;
        float* ac = acc + o * D;
        for (int d = 0; d < D; ++d) ac[d] = 0.0f;
        for (int j = j0; j < j1; ++j) {
          const float e = (s[j - j0] == -INFINITY) ? 0.0f : expf(s[j - j0] - mx);
          sum += e;
          const int64_t r = token_row(&a, b, h / G, j);
          if (r < 0) continue;
          for (int d = 0; d < D; ++d) ac[d] += e * load_elem(v_pool, pool_dtype, r + d);
        }
        m[o] = mx;
        l[o] = sum;
      }
    }
  }
  free(s);
  return 0;
}

int orc_splitk_merge(float* out, const float* m, const float* l, const float* acc,
                     const int32_t* ctx_lens, int max_blocks_per_seq, int block_size,
                     int num_seqs, int num_q_heads, int head_dim, int partition_size,
                     int max_parts) {
  if (!out || !m || !l || !acc || !ctx_lens || partition_size <= 0) return -1;
  const int D = head_dim;
  for (int b = 0; b < num_seqs; ++b) {
    const int L = clamp_ctx(ctx_lens[b], max_blocks_per_seq, block_size);
    const int np = (L + partition_size - 1) / partition_size;
    for (int h = 0; h < num_q_heads; ++h) {
      const int64_t base = ((int64_t)b * num_q_heads + h) * max_parts;
      float* o = out + ((int64_t)b * num_q_heads + h) * D;
      float M = -INFINITY;
      for (int p = 0; p < np; ++p) M = fmaxf(M, m[base + p]);
      for (int d = 0; d < D; ++d) o[d] = 0.0f;
      if (np == 0 || M == -INFINITY) continue;
      float den = 0.0f;
      for (int p = 0; p < np; ++p) {
        const float w = (m[base + p] == -INFINITY) ? 0.0f : expf(m[base + p] - M);
        den += w * l[base + p];
        for (int d = 0; d < D; ++d) o[d] += w * acc[(base + p) * D + d];
      }
      for (int d = 0; d < D; ++d) o[d] /= den;
    }
  }
  return 0;
}

/* ---- threaded baseline ------------------------------------------------- */

typedef struct {
  dec_args a;
  float* out;
  int num_seqs, next_unit_stride, first_unit, max_ctx;
} mt_job;

static void* mt_worker(void* p) {
  mt_job* j = (mt_job*)p;
  const dec_args* a = &j->a;
  const int G = a->num_q_heads / a->num_kv_heads;
  const int units = j->num_seqs * a->num_kv_heads;
  float* s = (float*)malloc(sizeof(float) * j->max_ctx);
  if (!s) return (void*)1;
  for (int u = j->first_unit; u < units; u += j->next_unit_stride) {
    const int b = u / a->num_kv_heads, kh = u % a->num_kv_heads;
    for (int g = 0; g < G; ++g) {
      const int h = kh * G + g;
      decode_one_f32(a, b, h, j->out + ((int64_t)b * a->num_q_heads + h) * a->head_dim, s);
    }
  }
  free(s);
  return NULL;
}

int orc_decode_attention_mt(float* out, const float* q, const void* k_pool, const void* v_pool,
                            const int32_t* block_tables, int max_blocks_per_seq,
                            const int32_t* ctx_lens, int num_seqs, int num_q_heads,
                            int num_kv_heads, int head_dim, int block_size, int64_t num_blocks,
                            float scale, int pool_dtype, int n_threads) {
  if (!out || n_threads <= 0 ||
      check_dec(q, k_pool, v_pool, block_tables, ctx_lens, num_q_heads, num_kv_heads, head_dim,
                block_size))
    return -1;
  if (n_threads > 1024) n_threads = 1024;
  dec_args a = {q, k_pool, v_pool, block_tables, ctx_lens, max_blocks_per_seq, num_q_heads,
                num_kv_heads, head_dim, block_size, pool_dtype, num_blocks, scale};
  const int mc = max_ctx_of(ctx_lens, num_seqs, max_blocks_per_seq, block_size);
  mt_job* jobs = (mt_job*)calloc(n_threads, sizeof(mt_job));
  pthread_t* th = (pthread_t*)calloc(n_threads, sizeof(pthread_t));
  if (!jobs || !th) {
    free(jobs);
    free(th);
    return -1;
  }
  int rc = 0;
  for (int t = 0; t < n_threads; ++t) {
    jobs[t] = (mt_job){a, out, num_seqs, n_threads, t, mc};
    if (pthread_create(&th[t], NULL, mt_worker, &jobs[t])) {
      n_threads = t;
      rc = -1;
      break;
    }
  }
  for (int t = 0; t < n_threads; ++t) {
    void* r = NULL;
    pthread_join(th[t], &r);
    if (r) rc = -1;
  }
  free(jobs);
  free(th);
  return rc;
}

/* ---- config-0 decoder ----------------------------------------------------- */

int64_t orc_decoder_param_count(const orc_decoder_config* c) {
  const int64_t d = c->d_model, V = c->vocab, f = c->d_ff;
  const int64_t kvd = (int64_t)c->n_kv_heads * (d / c->n_heads);
  const int64_t per_layer = 2 * d + (d * d + d) + 2 * (kvd * d + kvd) + (d * d + d) + 2 * d +
                            (f * d + f) + (d * f + d);
  return V * d + c->n_layers * per_layer + 2 * d + V * d;
}

void orc_linear(float* y, const float* x, const float* w, const float* b, int rows, int in_dim,
                int out_dim) {
  for (int r = 0; r < rows; ++r)
    for (int o = 0; o < out_dim; ++o) {
      float sum = 0.0f; /* sum += x * w, in order (lib.rs:519-525) */
      for (int i = 0; i < in_dim; ++i) sum += x[(int64_t)r * in_dim + i] * w[(int64_t)o * in_dim + i];
      y[(int64_t)r * out_dim + o] = b ? sum + b[o] : sum;
    }
}

void orc_layer_norm(float* y, const float* x, const float* g, const float* b, int rows, int dim,
                    float eps) {
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (int64_t)r * dim;
    float sum = 0.0f;
    for (int i = 0; i < dim; ++i) sum += xr[i];
    const float mean = sum / (float)dim;
    float vs = 0.0f;
    for (int i = 0; i < dim; ++i) {
      const float t = xr[i] - mean;
      vs += t * t; /* powi(2) */
    }
    const float var = vs / (float)dim;
    const float sd = sqrtf(var + eps);
    for (int i = 0; i < dim; ++i) y[(int64_t)r * dim + i] = (xr[i] - mean) / sd * g[i] + b[i];
  }
}

void orc_gelu(float* y, const float* x, int64_t n) {
  const float k = sqrtf(2.0f / 3.14159265358979323846f);
  for (int64_t i = 0; i < n; ++i) {
    const float v = x[i];
    const float x3 = v * v * v;
    const float xp = v + 0.044715f * x3;
    const float t = tanhf(k * xp);
    y[i] = 0.5f * v * (1.0f + t);
  }
}

void orc_positional_encoding(float* pe, int max_len, int d_model) {
  for (int pos = 0; pos < max_len; ++pos)
    for (int i = 0; i < d_model; ++i) {
      const float angle = (float)pos / powf(10000.0f, (float)(2 * (i / 2)) / (float)d_model);
      pe[(int64_t)pos * d_model + i] = (i % 2 == 0) ? sinf(angle) : cosf(angle);
    }
}

int orc_decoder_generate(const orc_decoder_config* c, const float* params,
                         const int32_t* prompt, int n_prompt, int n_new, int32_t* out_tokens,
                         float* out_logits) {
  if (!c || !params || !prompt || !out_tokens || n_prompt < 1 || n_new < 0) return -1;
  if (n_new == 0) return 0;
  const int d = c->d_model, V = c->vocab, f = c->d_ff, H = c->n_heads, Hk = c->n_kv_heads;
  if (d % H || H % Hk) return -1;
  const int dh = d / H, kvd = Hk * dh, G = H / Hk;
  const int total = n_prompt + (n_new > 0 ? n_new - 1 : 0);
  if (total > c->max_seq) return -1;
  const float scale = 1.0f / sqrtf((float)dh); /* tape_transformer.rs:75 */

  float* pe = malloc(sizeof(float) * (size_t)c->max_seq * d);
  float* kc = malloc(sizeof(float) * (size_t)c->n_layers * c->max_seq * kvd);
  float* vc = malloc(sizeof(float) * (size_t)c->n_layers * c->max_seq * kvd);
  float* x = malloc(sizeof(float) * d);
  float* h = malloc(sizeof(float) * d);
  float* q = malloc(sizeof(float) * d);
  float* o = malloc(sizeof(float) * d);
  float* a = malloc(sizeof(float) * d);
  float* ff = malloc(sizeof(float) * f);
  float* ff2 = malloc(sizeof(float) * f);
  float* s = malloc(sizeof(float) * c->max_seq);
  float* logits = malloc(sizeof(float) * V);
  if (!pe || !kc || !vc || !x || !h || !q || !o || !a || !ff || !ff2 || !s || !logits) return -1;
  orc_positional_encoding(pe, c->max_seq, d);

  int32_t cur = prompt[0];
  int produced = 0;
  for (int pos = 0; pos < total; ++pos) {
    const float* emb = params + (int64_t)cur * d;
    for (int i = 0; i < d; ++i) x[i] = emb[i] + pe[(int64_t)pos * d + i];
    const float* p = params + (int64_t)V * d;
    for (int l = 0; l < c->n_layers; ++l) {
      const float *ln1g = p, *ln1b = p + d;
      p += 2 * d;
      const float *wq = p, *bq = p + (int64_t)d * d;
      p += (int64_t)d * d + d;
      const float *wk = p, *bk = p + (int64_t)kvd * d;
      p += (int64_t)kvd * d + kvd;
      const float *wv = p, *bv = p + (int64_t)kvd * d;
      p += (int64_t)kvd * d + kvd;
      const float *wo = p, *bo = p + (int64_t)d * d;
      p += (int64_t)d * d + d;
      const float *ln2g = p, *ln2b = p + d;
      p += 2 * d;
      const float *w1 = p, *b1 = p + (int64_t)f * d;
      p += (int64_t)f * d + f;
      const float *w2 = p, *b2 = p + (int64_t)d * f;
      p += (int64_t)d * f + d;

      float* kl = kc + ((int64_t)l * c->max_seq + pos) * kvd;
      float* vl = vc + ((int64_t)l * c->max_seq + pos) * kvd;
      orc_layer_norm(h, x, ln1g, ln1b, 1, d, c->eps);
      orc_linear(q, h, wq, bq, 1, d, d);
      orc_linear(kl, h, wk, bk, 1, d, kvd);
      orc_linear(vl, h, wv, bv, 1, d, kvd);
      for (int hh = 0; hh < H; ++hh) { /* per head, as tape_transformer.rs:98-128 */
        const int kh = hh / G;
        float mx = -INFINITY;
        for (int j = 0; j <= pos; ++j) {
          const float* kj = kc + ((int64_t)l * c->max_seq + j) * kvd + kh * dh;
          float dot = 0.0f;
          for (int e = 0; e < dh; ++e) dot += q[hh * dh + e] * kj[e];
          s[j] = dot * scale;
          mx = fmaxf(mx, s[j]);
        }
        float sum = 0.0f;
        for (int j = 0; j <= pos; ++j) {
          s[j] = expf(s[j] - mx);
          sum += s[j];
        }
        const float inv = 1.0f / sum;
        for (int e = 0; e < dh; ++e) o[hh * dh + e] = 0.0f;
        for (int j = 0; j <= pos; ++j) {
          const float pj = s[j] * inv;
          const float* vj = vc + ((int64_t)l * c->max_seq + j) * kvd + kh * dh;
          for (int e = 0; e < dh; ++e) o[hh * dh + e] += pj * vj[e];
        }
      }
      orc_linear(a, o, wo, bo, 1, d, d);
      for (int i = 0; i < d; ++i) x[i] = x[i] + a[i];
      orc_layer_norm(h, x, ln2g, ln2b, 1, d, c->eps);
      orc_linear(ff, h, w1, b1, 1, d, f);
      orc_gelu(ff2, ff, f);
      orc_linear(a, ff2, w2, b2, 1, f, d);
      for (int i = 0; i < d; ++i) x[i] = x[i] + a[i];
    }
    const float *lnfg = p, *lnfb = p + d, *wlm = p + 2 * d;
    if (pos + 1 < n_prompt) {
      cur = prompt[pos + 1];
      continue;
    }
    orc_layer_norm(h, x, lnfg, lnfb, 1, d, c->eps);
    orc_linear(logits, h, wlm, NULL, 1, d, V);
    const int32_t next = (int32_t)orc_argmax(logits, V);
    if (out_logits) memcpy(out_logits + (int64_t)produced * V, logits, sizeof(float) * V);
    out_tokens[produced++] = next;
    cur = next;
  }
  free(pe); free(kc); free(vc); free(x); free(h); free(q); free(o); free(a);
  free(ff); free(ff2); free(s); free(logits);
  return 0;
}
