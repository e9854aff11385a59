// model_ops.hpp -- internal entry of model_ops.hip shared by the decoder and
// the serving engine.
#pragma once

#include "common.hpp"

namespace rkv {

// rkv_linear with a fused epilogue: epi 0 y = x W^T + b; 1 y = res + (x W^T + b)
// (residual add, y may alias res); 2 y = gelu(x W^T + b).  The same
// arithmetic, in the same order, as rkv_linear followed by rkv_add / rkv_gelu.
int linear_launch(float* y, const float* x, const float* w, const float* b, const float* res,
                  int epi, int rows, int in_dim, int out_dim, hipStream_t s);

}  // namespace rkv
