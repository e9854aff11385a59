// model_ops.hip -- the fp32 TensorOps subset a decoder step needs on gfx950
// (include/rustral_model.h): embedding + positional term, linear, layer norm,
// gelu, add, argmax.
//
// These are not the hot path (the KV cache and decode attention are); they
// exist so a whole decoder step runs on the device.  Each op keeps the
// reference's summation order: one thread owns one output and adds its terms
// serially, with floating-point contraction off, so the results are the bits
// the ndarray backend computes (except gelu's tanh, from the device library).
#include "common.hpp"

#include <cmath>

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

// One thread per output; the dot product runs serially over in_dim.
__global__ __launch_bounds__(64) void linear_kernel(float* __restrict__ y,
                                                    const float* __restrict__ x,
                                                    const float* __restrict__ w,
                                                    const float* __restrict__ b, int rows,
                                                    int in_dim, int out_dim) {
#pragma clang fp contract(off)
  const int o = blockIdx.x * blockDim.x + threadIdx.x;
  const int r = blockIdx.y;
  if (o >= out_dim || r >= rows) return;
  const float* xr = x + (int64_t)r * in_dim;
  const float* wo = w + (int64_t)o * in_dim;
  float sum = 0.0f;
  for (int i = 0; i < in_dim; ++i) sum += xr[i] * wo[i];
  y[(int64_t)r * out_dim + o] = b ? sum + b[o] : sum;
}

// One wave per row: lane 0 forms the serial sums, every lane writes outputs.
__global__ __launch_bounds__(64) void layer_norm_kernel(float* __restrict__ y,
                                                        const float* __restrict__ x,
                                                        const float* __restrict__ g,
                                                        const float* __restrict__ b, int rows,
                                                        int dim, float eps) {
#pragma clang fp contract(off)
  __shared__ float s_stat[2];
  const int r = blockIdx.x, lane = threadIdx.x;
  if (r >= rows) return;
  const float* xr = x + (int64_t)r * dim;
  if (lane == 0) {
    float sum = 0.0f;
    for (int i = 0; i < dim; ++i) sum += xr[i];
    const float mean = sum / (float)dim;
    float vs = 0.0f;
    for (int i = 0; i < dim; ++i) {
      const float t = xr[i] - mean;
      vs += t * t;
    }
    s_stat[0] = mean;
    s_stat[1] = sqrtf(vs / (float)dim + eps);
  }
  __syncthreads();
  const float mean = s_stat[0], sd = s_stat[1];
  for (int i = lane; i < dim; i += 64) y[(int64_t)r * dim + i] = (xr[i] - mean) / sd * g[i] + b[i];
}

__global__ __launch_bounds__(256) void gelu_kernel(float* __restrict__ y,
                                                   const float* __restrict__ x, int64_t n) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float k = sqrtf(2.0f / 3.14159265358979323846f);
  const float v = x[i];
  const float x3 = v * v * v;
  const float xp = v + 0.044715f * x3;
  const float t = tanhf(k * xp);
  y[i] = 0.5f * v * (1.0f + t);
}

// y may alias a or b (in-place residual add)
__global__ __launch_bounds__(256) void add_kernel(float* y, const float* a, const float* b,
                                                  int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = a[i] + b[i];
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

unsigned blocks_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace
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
  if (rows < 0 || in_dim <= 0 || out_dim <= 0)
    return fail(RKV_ERR_INVALID_ARG, "rkv_linear: bad size argument");
  if (rows == 0) return RKV_OK;
  if (rows > 65535) return fail(RKV_ERR_INVALID_ARG, "rkv_linear: rows must be <= 65535");
  if (!y || !x || !w) return fail(RKV_ERR_INVALID_ARG, "rkv_linear: null pointer argument");
  linear_kernel<<<dim3(blocks_for(out_dim, 64), (unsigned)rows), 64, 0,
                  static_cast<hipStream_t>(stream)>>>(y, x, w, b, rows, in_dim, out_dim);
  return check_launch("rkv_linear");
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

extern "C" int rkv_argmax(int32_t* out, const float* x, int rows, int n, void* stream) {
  clear_error();
  if (rows < 0 || n <= 0) return fail(RKV_ERR_INVALID_ARG, "rkv_argmax: bad size argument");
  if (rows == 0) return RKV_OK;
  if (!out || !x) return fail(RKV_ERR_INVALID_ARG, "rkv_argmax: null pointer argument");
  argmax_kernel<<<(unsigned)rows, 64, 0, static_cast<hipStream_t>(stream)>>>(out, x, rows, n);
  return check_launch("rkv_argmax");
}
