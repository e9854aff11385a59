// model_ops.hip -- the fp32 TensorOps subset a decoder step needs on gfx950
// (include/rustral_model.h): embedding + positional term, linear, layer norm,
// gelu, add, argmax, and the per-head attention recipe's matmul, transpose,
// mul_scalar and softmax_dim.
//
// These are not the hot path (the KV cache and decode attention are); they
// exist so a whole decoder step runs on the device.  Each op keeps the
// reference's summation order: one thread owns one output and adds its terms
// serially, with floating-point contraction off, so the results are the bits
// the ndarray backend computes (except gelu's tanh, from the device library).
#include "model_ops.hpp"

#include <cmath>
#include <type_traits>

namespace rkv {
namespace {

__global__ __launch_bounds__(256) void embed_kernel(float* __restrict__ out,
                                                    const float* __restrict__ table,
                                                    const int32_t* __restrict__ ids,
                                                    const float* __restrict__ pe,
                                                    const int32_t* __restrict__ positions,
                                                    int n_tokens, int vocab, int dim,
                                                    int max_len) {
#pragma clang fp contract(off)
  const int t = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_tokens || i >= dim) return;
  const int id = ids[t];
  float v = NAN;
  if (id >= 0 && id < vocab) {
    v = table[(int64_t)id * dim + i];
    if (pe) {
      const int p = positions[t];
      v = (p >= 0 && p < max_len) ? v + pe[(int64_t)p * dim + i] : NAN;
    }
  }
  out[(int64_t)t * dim + i] = v;
}

// One thread per output; the dot product runs serially over in_dim (the
// reference's order).  The input row is staged in LDS (coalesced) and each
// thread reads its weight row four floats at a time, so the serial sum is not
// waiting on scattered scalar loads.  EPI: 0 y = sum + b; 1 y = res + (sum + b)
// (a fused residual add; y may be res); 2 y = gelu(sum + b).
constexpr int kMaxStagedIn = 8192;  // floats of the input row kept in LDS

__device__ __forceinline__ float gelu_f(float v) {
#pragma clang fp contract(off)
  const float k = sqrtf(2.0f / 3.14159265358979323846f);
  const float x3 = v * v * v;
  const float xp = v + 0.044715f * x3;
  const float t = tanhf(k * xp);
  return 0.5f * v * (1.0f + t);
}

// Stages the n floats of row xr in s_x (64 threads); with LN the row is then
// layer-normed in place exactly as layer_norm_kernel does it (lane 0's serial
// sums, the same expression per element), so the staged values are the bits
// rkv_layer_norm writes.
template <bool LN>
__device__ __forceinline__ void stage_row(float* s_x, float* s_stat, const float* xr, int n,
                                          const float* __restrict__ ln_g,
                                          const float* __restrict__ ln_b, float eps) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x;
  for (int i = lane; i < n; i += 64) s_x[i] = xr[i];
  __syncthreads();
  if constexpr (LN) {
    if (lane == 0) {
      float sum = 0.0f;
      for (int i = 0; i < n; ++i) sum += s_x[i];
      const float mean = sum / (float)n;
      float vs = 0.0f;
      for (int i = 0; i < n; ++i) {
        const float t = s_x[i] - mean;
        vs += t * t;
      }
      s_stat[0] = mean;
      s_stat[1] = sqrtf(vs / (float)n + eps);
    }
    __syncthreads();
    const float mean = s_stat[0], sd = s_stat[1];
    for (int i = lane; i < n; i += 64) s_x[i] = (s_x[i] - mean) / sd * ln_g[i] + ln_b[i];
    __syncthreads();
  }
}

// LN: the input row is layer-normed first (ln_g, ln_b, eps), as rkv_layer_norm
// followed by the linear.
template <int EPI, bool VEC, bool LN>
__global__ __launch_bounds__(64) void linear_kernel(float* y, const float* __restrict__ x,
                                                    const float* __restrict__ w,
                                                    const float* __restrict__ b, const float* res,
                                                    int rows, int in_dim, int out_dim,
                                                    const float* __restrict__ ln_g,
                                                    const float* __restrict__ ln_b, float eps) {
#pragma clang fp contract(off)
  __shared__ float s_x[kMaxStagedIn];
  __shared__ float s_stat[2];
  const int o = blockIdx.x * blockDim.x + threadIdx.x;
  const int r = blockIdx.y;
  stage_row<LN>(s_x, s_stat, x + (int64_t)r * in_dim, in_dim, ln_g, ln_b, eps);
  if (o >= out_dim || r >= rows) return;
  const float* wo = w + (int64_t)o * in_dim;
  float sum = 0.0f;
  if constexpr (VEC) {  // in_dim % 4 == 0 and w 16-byte aligned
#pragma unroll 8
    for (int i = 0; i < in_dim; i += 4) {
      const float4 wv = *reinterpret_cast<const float4*>(wo + i);
      sum += s_x[i] * wv.x;
      sum += s_x[i + 1] * wv.y;
      sum += s_x[i + 2] * wv.z;
      sum += s_x[i + 3] * wv.w;
    }
  } else {
    for (int i = 0; i < in_dim; ++i) sum += s_x[i] * wo[i];
  }
  const int64_t at = (int64_t)r * out_dim + o;
  const float v = b ? sum + b[o] : sum;
  if constexpr (EPI == 1)
    y[at] = res[at] + v;
  else if constexpr (EPI == 2)
    y[at] = gelu_f(v);
  else
    y[at] = v;
}

// One wave per row: the row is staged in LDS, lane 0 forms the serial sums
// from it, every lane writes outputs.
__global__ __launch_bounds__(64) void layer_norm_kernel(float* __restrict__ y,
                                                        const float* __restrict__ x,
                                                        const float* __restrict__ g,
                                                        const float* __restrict__ b, int rows,
                                                        int dim, float eps) {
#pragma clang fp contract(off)
  __shared__ float s_stat[2];
  __shared__ float s_row[8192];
  const int r = blockIdx.x, lane = threadIdx.x;
  if (r >= rows) return;
  const float* xr = x + (int64_t)r * dim;
  for (int i = lane; i < dim; i += 64) s_row[i] = xr[i];
  __syncthreads();
  if (lane == 0) {
    float sum = 0.0f;
    for (int i = 0; i < dim; ++i) sum += s_row[i];
    const float mean = sum / (float)dim;
    float vs = 0.0f;
    for (int i = 0; i < dim; ++i) {
      const float t = s_row[i] - mean;
      vs += t * t;
    }
    s_stat[0] = mean;
    s_stat[1] = sqrtf(vs / (float)dim + eps);
  }
  __syncthreads();
  const float mean = s_stat[0], sd = s_stat[1];
  for (int i = lane; i < dim; i += 64) y[(int64_t)r * dim + i] = (s_row[i] - mean) / sd * g[i] + b[i];
}

__global__ __launch_bounds__(256) void gelu_kernel(float* __restrict__ y,
                                                   const float* __restrict__ x, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  y[i] = gelu_f(x[i]);
}

// y may alias a or b (in-place residual add)
__global__ __launch_bounds__(256) void add_kernel(float* y, const float* a, const float* b,
                                                  int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = a[i] + b[i];
}

__global__ __launch_bounds__(256) void mul_scalar_kernel(float* y, const float* x, float s,
                                                         int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = x[i] * s;
}

// Softmax along an axis of `axis` elements at stride `inner` (CpuOps::
// softmax_dim's loops): max over the line with NaN skipped (f32::max /
// fmaxf), e = exp(x - max) written out and added serially in axis order,
// then every e scaled by 1 / sum.
//
// Strided lines (inner > 1): one thread per line, lanes on consecutive i, so
// every step of the three serial loops is a coalesced row access.
__global__ __launch_bounds__(256) void softmax_strided_kernel(float* y, const float* x,
                                                              int64_t lines, int64_t axis,
                                                              int64_t inner) {
#pragma clang fp contract(off)
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= lines) return;
  const int64_t o = g / inner, i = g - o * inner;
  const float* xl = x + o * axis * inner + i;
  float* yl = y + o * axis * inner + i;
  float mx = -INFINITY;
  for (int64_t a = 0; a < axis; ++a) mx = fmaxf(mx, xl[a * inner]);
  float sum = 0.0f;
  for (int64_t a = 0; a < axis; ++a) {
    const float e = expf(xl[a * inner] - mx);
    yl[a * inner] = e;
    sum += e;
  }
  const float inv = 1.0f / sum;
  for (int64_t a = 0; a < axis; ++a) yl[a * inner] *= inv;
}

// Contiguous lines (inner == 1): one 256-thread workgroup per row.  The max
// is a tree over the workgroup (max is exact, so any order gives the serial
// scan's value); the exps are computed in parallel, kChunk at a time, into
// LDS and y, and lane 0 adds each chunk in index order, so the sum is the
// reference's serial sum.  Each thread scales the entries it wrote itself.
constexpr int kSoftmaxChunk = 2048;

__global__ __launch_bounds__(256) void softmax_rows_kernel(float* y, const float* x,
                                                           int64_t axis) {
#pragma clang fp contract(off)
  __shared__ float s_e[kSoftmaxChunk];
  __shared__ float s_red[4];
  __shared__ float s_sum;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const float* xr = x + (int64_t)blockIdx.x * axis;
  float* yr = y + (int64_t)blockIdx.x * axis;
  float mx = -INFINITY;
  for (int64_t a = t; a < axis; a += 256) mx = fmaxf(mx, xr[a]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) s_red[w] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  float sum = 0.0f;  // lane 0 of wave 0 only
  for (int64_t c0 = 0; c0 < axis; c0 += kSoftmaxChunk) {
    const int n = (int)((axis - c0) < kSoftmaxChunk ? (axis - c0) : kSoftmaxChunk);
    for (int j = t; j < n; j += 256) {
      const float e = expf(xr[c0 + j] - mx);
      s_e[j] = e;
      yr[c0 + j] = e;
    }
    __syncthreads();
    if (t == 0)
      for (int j = 0; j < n; ++j) sum += s_e[j];
    __syncthreads();
  }
  if (t == 0) s_sum = sum;
  __syncthreads();
  const float inv = 1.0f / s_sum;
  for (int64_t c0 = 0; c0 < axis; c0 += kSoftmaxChunk) {
    const int n = (int)((axis - c0) < kSoftmaxChunk ? (axis - c0) : kSoftmaxChunk);
    for (int j = t; j < n; j += 256) yr[c0 + j] *= inv;
  }
}

// y[m][n] = sum_k a[m][k] * b[k][n], the sum serial in k (the reference's
// naive loop order) and without contraction.  16 x 16 outputs per workgroup,
// one per thread; k advances through 16-wide tiles of a and b staged in LDS.
constexpr int kMmTile = 16;

__global__ __launch_bounds__(256) void matmul_kernel(float* __restrict__ y,
                                                     const float* __restrict__ a,
                                                     const float* __restrict__ b, int m, int k,
                                                     int n) {
#pragma clang fp contract(off)
  __shared__ float s_a[kMmTile][kMmTile + 1];
  __shared__ float s_b[kMmTile][kMmTile + 1];
  const int tx = threadIdx.x & (kMmTile - 1), ty = threadIdx.x / kMmTile;
  const int row = blockIdx.y * kMmTile + ty, col = blockIdx.x * kMmTile + tx;
  float sum = 0.0f;
  for (int k0 = 0; k0 < k; k0 += kMmTile) {
    s_a[ty][tx] = (row < m && k0 + tx < k) ? a[(int64_t)row * k + k0 + tx] : 0.0f;
    s_b[ty][tx] = (k0 + ty < k && col < n) ? b[(int64_t)(k0 + ty) * n + col] : 0.0f;
    __syncthreads();
    const int kt = (k - k0) < kMmTile ? (k - k0) : kMmTile;
    for (int j = 0; j < kt; ++j) sum += s_a[ty][j] * s_b[j][tx];
    __syncthreads();
  }
  if (row < m && col < n) y[(int64_t)row * n + col] = sum;
}

// y[n][m] = x[m][n]: 32 x 32 tiles through LDS (one padding column keeps the
// transposed reads off a single bank), both sides coalesced.
__global__ __launch_bounds__(256) void transpose_kernel(float* __restrict__ y,
                                                        const float* __restrict__ x, int m,
                                                        int n) {
  __shared__ float s_t[32][33];
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8 threads
  const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
  for (int r = ty; r < 32; r += 8)
    if (r0 + r < m && c0 + tx < n) s_t[r][tx] = x[(int64_t)(r0 + r) * n + c0 + tx];
  __syncthreads();
  for (int c = ty; c < 32; c += 8)
    if (c0 + c < n && r0 + tx < m) y[(int64_t)(c0 + c) * m + r0 + tx] = s_t[tx][c];
}

// One wave per row.  Without NaN: each lane scans its elements (i = lane,
// lane + 64, ...) keeping the last maximum, then lanes combine (larger value,
// or the larger index on a tie).  With a NaN anywhere the answer depends on
// the scan order, so lane 0 repeats the reference's left-to-right scan.
__global__ __launch_bounds__(64) void argmax_kernel(int32_t* __restrict__ out,
                                                    const float* __restrict__ x, int rows,
                                                    int n) {
  const int r = blockIdx.x, lane = threadIdx.x;
  if (r >= rows) return;
  const float* xr = x + (int64_t)r * n;
  bool nan = false;
  float bv = -INFINITY;
  int bi = -1;
  for (int i = lane; i < n; i += 64) {
    const float v = xr[i];
    nan |= v != v;
    if (bi < 0 || v >= bv) {
      bv = v;
      bi = i;
    }
  }
  if (__ballot(nan)) {
    if (lane == 0) {
      int best = 0;
      for (int i = 1; i < n; ++i)
        if (!(xr[best] > xr[i])) best = i;
      out[r] = best;
    }
    return;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi > bi))) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) out[r] = bi;
}

// The attention input of one decoder layer in one launch: LN1 of the token's
// row, its q / k / v projections, and the K / V rows appended to the paged
// pools.  grid = (columns of [q | k | v] / 64, tokens); one thread per column.
// The row is normalised in LDS by stage_row and every column's dot product
// runs serially in linear_kernel's order, so q and the pool rows are
// the bits of rkv_layer_norm + 3 x rkv_linear + rkv_append.  K / V columns go
// straight to slot_mapping[t]'s pool row (bf16 pools: round to nearest even,
// as rkv_append); a slot outside the pool appends nothing.
template <bool LN, bool VEC, bool BF16>
__global__ __launch_bounds__(64) void qkv_append_kernel(
    float* __restrict__ q_out, void* __restrict__ k_pool, void* __restrict__ v_pool,
    const int64_t* __restrict__ slot_mapping, const float* __restrict__ x,
    const float* __restrict__ ln_g, const float* __restrict__ ln_b, float eps,
    const float* __restrict__ wq, const float* __restrict__ bq, const float* __restrict__ wk,
    const float* __restrict__ bk, const float* __restrict__ wv, const float* __restrict__ bv,
    int d_model, int q_dim, int num_kv_heads, int head_dim, int block_size, int64_t num_slots) {
#pragma clang fp contract(off)
  __shared__ float s_x[kMaxStagedIn];
  __shared__ float s_stat[2];
  const int r = blockIdx.y, lane = threadIdx.x;
  stage_row<LN>(s_x, s_stat, x + (int64_t)r * d_model, d_model, ln_g, ln_b, eps);
  const int kvd = num_kv_heads * head_dim;
  const int o = blockIdx.x * 64 + lane;
  if (o >= q_dim + 2 * kvd) return;
  const int part = o < q_dim ? 0 : (o < q_dim + kvd ? 1 : 2);  // q, k or v
  const int col = part == 0 ? o : (part == 1 ? o - q_dim : o - q_dim - kvd);
  const float* w = part == 0 ? wq : (part == 1 ? wk : wv);
  const float* b = part == 0 ? bq : (part == 1 ? bk : bv);
  const float* wo = w + (int64_t)col * d_model;
  float sum = 0.0f;
  if constexpr (VEC) {  // d_model % 4 == 0 and the weights 16-byte aligned
#pragma unroll 8
    for (int i = 0; i < d_model; i += 4) {
      const float4 wv4 = *reinterpret_cast<const float4*>(wo + i);
      sum += s_x[i] * wv4.x;
      sum += s_x[i + 1] * wv4.y;
      sum += s_x[i + 2] * wv4.z;
      sum += s_x[i + 3] * wv4.w;
    }
  } else {
    for (int i = 0; i < d_model; ++i) sum += s_x[i] * wo[i];
  }
  const float v = b ? sum + b[col] : sum;
  if (part == 0) {
    q_out[(int64_t)r * q_dim + col] = v;
    return;
  }
  const int64_t slot = slot_mapping[r];
  if (slot < 0 || slot >= num_slots) return;  // padding or out-of-range slot
  const int64_t blk = slot / block_size, row = slot - blk * block_size;
  const int h = col / head_dim, e = col - h * head_dim;
  const int64_t dst = ((blk * num_kv_heads + h) * block_size + row) * head_dim + e;
  void* pool = part == 1 ? k_pool : v_pool;
  if constexpr (BF16)
    static_cast<uint16_t*>(pool)[dst] = (uint16_t)bf16_rne(v);
  else
    static_cast<float*>(pool)[dst] = v;
}

unsigned blocks_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

// Shared by rkv_linear and the decoder / engine (fused epilogues).
int linear_launch(float* y, const float* x, const float* w, const float* b, const float* res,
                  int epi, int rows, int in_dim, int out_dim, hipStream_t s, const float* ln_g,
                  const float* ln_b, float eps) {
  if (rows < 0 || in_dim <= 0 || out_dim <= 0)
    return fail(RKV_ERR_INVALID_ARG, "rkv_linear: bad size argument");
  if (rows == 0) return RKV_OK;
  if (rows > 65535) return fail(RKV_ERR_INVALID_ARG, "rkv_linear: rows must be <= 65535");
  if (in_dim > kMaxStagedIn) return fail(RKV_ERR_UNSUPPORTED, "rkv_linear: in_dim must be <= 8192");
  if (!y || !x || !w || (epi == 1 && !res))
    return fail(RKV_ERR_INVALID_ARG, "rkv_linear: null pointer argument");
  if (!ln_g != !ln_b) return fail(RKV_ERR_INVALID_ARG, "rkv_linear: ln_g and ln_b go together");
  const bool vec = in_dim % 4 == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0;
  const dim3 grid(blocks_for(out_dim, 64), (unsigned)rows);
  // one instantiation per (epilogue, weight loads, layer norm)
  auto go = [&](auto epi_c, auto ln_c) {
    constexpr int E = decltype(epi_c)::value;
    constexpr bool L = decltype(ln_c)::value;
    if (vec)
      linear_kernel<E, true, L><<<grid, 64, 0, s>>>(y, x, w, b, res, rows, in_dim, out_dim, ln_g,
                                                    ln_b, eps);
    else
      linear_kernel<E, false, L><<<grid, 64, 0, s>>>(y, x, w, b, res, rows, in_dim, out_dim, ln_g,
                                                     ln_b, eps);
  };
  auto with_epi = [&](auto ln_c) {
    if (epi == 1)
      go(std::integral_constant<int, 1>{}, ln_c);
    else if (epi == 2)
      go(std::integral_constant<int, 2>{}, ln_c);
    else
      go(std::integral_constant<int, 0>{}, ln_c);
  };
  if (ln_g)
    with_epi(std::true_type{});
  else
    with_epi(std::false_type{});
  return check_launch("rkv_linear");
}

}  // namespace rkv

using namespace rkv;

extern "C" int rkv_embed(float* out, const float* table, const int32_t* ids, const float* pe,
                         const int32_t* positions, int n_tokens, int vocab, int dim, int max_len,
                         void* stream) {
  clear_error();
  if (n_tokens < 0 || vocab <= 0 || dim <= 0 || (pe && max_len <= 0))
    return fail(RKV_ERR_INVALID_ARG, "rkv_embed: bad size argument");
  if (n_tokens == 0) return RKV_OK;
  if (n_tokens > 65535) return fail(RKV_ERR_INVALID_ARG, "rkv_embed: n_tokens must be <= 65535");
  if (!out || !table || !ids || (pe && !positions))
    return fail(RKV_ERR_INVALID_ARG, "rkv_embed: null pointer argument");
  embed_kernel<<<dim3(blocks_for(dim, 256), (unsigned)n_tokens), 256, 0,
                 static_cast<hipStream_t>(stream)>>>(out, table, ids, pe, positions, n_tokens,
                                                     vocab, dim, max_len);
  return check_launch("rkv_embed");
}

extern "C" int rkv_linear(float* y, const float* x, const float* w, const float* b, int rows,
                          int in_dim, int out_dim, void* stream) {
  clear_error();
  return linear_launch(y, x, w, b, nullptr, 0, rows, in_dim, out_dim,
                       static_cast<hipStream_t>(stream));
}

extern "C" int rkv_qkv_append(float* q_out, void* k_pool, void* v_pool,
                              const int64_t* slot_mapping, const float* x, const float* ln_g,
                              const float* ln_b, float eps, const float* wq, const float* bq,
                              const float* wk, const float* bk, const float* wv,
                              const float* bv, int n_tokens, int d_model, int q_dim,
                              int num_kv_heads, int head_dim, int block_size,
                              int64_t num_blocks, int dtype, void* stream) {
  clear_error();
  if (n_tokens < 0 || d_model <= 0 || q_dim <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      block_size <= 0 || num_blocks <= 0)
    return fail(RKV_ERR_INVALID_ARG, "rkv_qkv_append: bad size argument");
  if (d_model > kMaxStagedIn)
    return fail(RKV_ERR_UNSUPPORTED, "rkv_qkv_append: d_model must be <= 8192");
  if (n_tokens > 65535)
    return fail(RKV_ERR_INVALID_ARG, "rkv_qkv_append: n_tokens must be <= 65535");
  if ((int64_t)q_dim + 2 * (int64_t)num_kv_heads * head_dim > (int64_t)INT32_MAX - 64)
    return fail(RKV_ERR_INVALID_ARG, "rkv_qkv_append: too many output columns");
  if (dtype != RKV_F32 && dtype != RKV_BF16)
    return fail(RKV_ERR_UNSUPPORTED, "rkv_qkv_append: pools must be RKV_F32 or RKV_BF16");
  if (!ln_g != !ln_b)
    return fail(RKV_ERR_INVALID_ARG, "rkv_qkv_append: ln_g and ln_b are both given or both NULL");
  if (n_tokens == 0) return RKV_OK;
  if (!q_out || !k_pool || !v_pool || !slot_mapping || !x || !wq || !wk || !wv)
    return fail(RKV_ERR_INVALID_ARG, "rkv_qkv_append: null pointer argument");
  const auto a16 = [](const float* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  const bool vec = d_model % 4 == 0 && a16(wq) && a16(wk) && a16(wv);
  const int cols = q_dim + 2 * num_kv_heads * head_dim;
  const dim3 grid(blocks_for(cols, 64), (unsigned)n_tokens);
  const int64_t num_slots = num_blocks * block_size;
  hipStream_t s = static_cast<hipStream_t>(stream);
#define RKV_QKV(LN, V, B)                                                                     \
  qkv_append_kernel<LN, V, B><<<grid, 64, 0, s>>>(q_out, k_pool, v_pool, slot_mapping, x, ln_g, \
                                                  ln_b, eps, wq, bq, wk, bk, wv, bv, d_model,  \
                                                  q_dim, num_kv_heads, head_dim, block_size,   \
                                                  num_slots)
  const bool ln = ln_g != nullptr, bf = dtype == RKV_BF16;
  if (ln) {
    if (vec) { if (bf) RKV_QKV(true, true, true); else RKV_QKV(true, true, false); }
    else { if (bf) RKV_QKV(true, false, true); else RKV_QKV(true, false, false); }
  } else {
    if (vec) { if (bf) RKV_QKV(false, true, true); else RKV_QKV(false, true, false); }
    else { if (bf) RKV_QKV(false, false, true); else RKV_QKV(false, false, false); }
  }
#undef RKV_QKV
  return check_launch("rkv_qkv_append");
}

extern "C" int rkv_layer_norm(float* y, const float* x, const float* g, const float* b, int rows,
                              int dim, float eps, void* stream) {
  clear_error();
  if (rows < 0 || dim <= 0 || dim > 8192)
    return fail(RKV_ERR_INVALID_ARG, "rkv_layer_norm: bad size argument");
  if (rows == 0) return RKV_OK;
  if (!y || !x || !g || !b) return fail(RKV_ERR_INVALID_ARG, "rkv_layer_norm: null pointer");
  layer_norm_kernel<<<(unsigned)rows, 64, 0, static_cast<hipStream_t>(stream)>>>(y, x, g, b, rows,
                                                                               dim, eps);
  return check_launch("rkv_layer_norm");
}

extern "C" int rkv_gelu(float* y, const float* x, int64_t n, void* stream) {
  clear_error();
  if (n < 0) return fail(RKV_ERR_INVALID_ARG, "rkv_gelu: n < 0");
  if (n == 0) return RKV_OK;
  if (!y || !x) return fail(RKV_ERR_INVALID_ARG, "rkv_gelu: null pointer argument");
  gelu_kernel<<<blocks_for(n, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(y, x, n);
  return check_launch("rkv_gelu");
}

extern "C" int rkv_add(float* y, const float* a, const float* b, int64_t n, void* stream) {
  clear_error();
  if (n < 0) return fail(RKV_ERR_INVALID_ARG, "rkv_add: n < 0");
  if (n == 0) return RKV_OK;
  if (!y || !a || !b) return fail(RKV_ERR_INVALID_ARG, "rkv_add: null pointer argument");
  add_kernel<<<blocks_for(n, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(y, a, b, n);
  return check_launch("rkv_add");
}

extern "C" int rkv_mul_scalar(float* y, const float* x, float s, int64_t n, void* stream) {
  clear_error();
  if (n < 0) return fail(RKV_ERR_INVALID_ARG, "rkv_mul_scalar: n < 0");
  if (n == 0) return RKV_OK;
  if (!y || !x) return fail(RKV_ERR_INVALID_ARG, "rkv_mul_scalar: null pointer argument");
  if (n > (int64_t)INT32_MAX * 256) return fail(RKV_ERR_INVALID_ARG, "rkv_mul_scalar: n too large");
  mul_scalar_kernel<<<blocks_for(n, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(y, x, s, n);
  return check_launch("rkv_mul_scalar");
}

extern "C" int rkv_softmax_dim(float* y, const float* x, int64_t outer, int64_t axis,
                               int64_t inner, void* stream) {
  clear_error();
  if (outer < 0 || inner < 0 || axis <= 0)
    return fail(RKV_ERR_INVALID_ARG, "rkv_softmax_dim: bad size argument (axis size must be > 0)");
  if (outer == 0 || inner == 0) return RKV_OK;
  if (!y || !x) return fail(RKV_ERR_INVALID_ARG, "rkv_softmax_dim: null pointer argument");
  if (outer > INT64_MAX / axis || outer * axis > INT64_MAX / inner)
    return fail(RKV_ERR_INVALID_ARG, "rkv_softmax_dim: element count overflows int64");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (inner == 1) {
    if (outer > INT32_MAX) return fail(RKV_ERR_INVALID_ARG, "rkv_softmax_dim: too many rows");
    softmax_rows_kernel<<<(unsigned)outer, 256, 0, s>>>(y, x, axis);
  } else {
    const int64_t lines = outer * inner;
    if (lines > (int64_t)INT32_MAX * 256)
      return fail(RKV_ERR_INVALID_ARG, "rkv_softmax_dim: too many lines");
    softmax_strided_kernel<<<blocks_for(lines, 256), 256, 0, s>>>(y, x, lines, axis, inner);
  }
  return check_launch("rkv_softmax_dim");
}

extern "C" int rkv_matmul(float* y, const float* a, const float* b, int m, int k, int n,
                          void* stream) {
  clear_error();
  if (m < 0 || k < 0 || n < 0) return fail(RKV_ERR_INVALID_ARG, "rkv_matmul: bad size argument");
  if (m == 0 || n == 0) return RKV_OK;
  if (!y || (k > 0 && (!a || !b)))
    return fail(RKV_ERR_INVALID_ARG, "rkv_matmul: null pointer argument");
  if ((m + kMmTile - 1) / kMmTile > 65535)
    return fail(RKV_ERR_INVALID_ARG, "rkv_matmul: m must be <= 1048560");
  const dim3 grid(blocks_for(n, kMmTile), (unsigned)((m + kMmTile - 1) / kMmTile));
  matmul_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(y, a, b, m, k, n);
  return check_launch("rkv_matmul");
}

extern "C" int rkv_transpose(float* y, const float* x, int m, int n, void* stream) {
  clear_error();
  if (m < 0 || n < 0) return fail(RKV_ERR_INVALID_ARG, "rkv_transpose: bad size argument");
  if (m == 0 || n == 0) return RKV_OK;
  if (!y || !x) return fail(RKV_ERR_INVALID_ARG, "rkv_transpose: null pointer argument");
  if (y == x) return fail(RKV_ERR_INVALID_ARG, "rkv_transpose: y must not alias x");
  if ((m + 31) / 32 > 65535) return fail(RKV_ERR_INVALID_ARG, "rkv_transpose: m must be <= 2097120");
  const dim3 grid(blocks_for(n, 32), (unsigned)((m + 31) / 32));
  transpose_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(y, x, m, n);
  return check_launch("rkv_transpose");
}

extern "C" int rkv_argmax(int32_t* out, const float* x, int rows, int n, void* stream) {
  clear_error();
  if (rows < 0 || n <= 0) return fail(RKV_ERR_INVALID_ARG, "rkv_argmax: bad size argument");
  if (rows == 0) return RKV_OK;
  if (!out || !x) return fail(RKV_ERR_INVALID_ARG, "rkv_argmax: null pointer argument");
  argmax_kernel<<<(unsigned)rows, 64, 0, static_cast<hipStream_t>(stream)>>>(out, x, rows, n);
  return check_launch("rkv_argmax");
}
