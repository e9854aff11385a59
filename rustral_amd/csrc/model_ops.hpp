// model_ops.hpp -- internal entry of model_ops.hip shared by the decoder and
// the serving engine.
#pragma once

#include "common.hpp"

namespace rkv {

// rkv_linear with a fused epilogue: epi 0 y = x W^T + b; 1 y = res + (x W^T + b)
// (residual add, y may alias res); 2 y = gelu(x W^T + b).  With ln_g / ln_b
// the input rows are layer-normed first (eps).  The same arithmetic, in the
// same order, as rkv_layer_norm, rkv_linear and then rkv_add / rkv_gelu.
int linear_launch(float* y, const float* x, const float* w, const float* b, const float* res,
                  int epi, int rows, int in_dim, int out_dim, hipStream_t s,
                  const float* ln_g = nullptr, const float* ln_b = nullptr, float eps = 0.0f);

}  // namespace rkv
