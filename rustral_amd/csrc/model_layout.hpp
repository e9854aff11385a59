// model_layout.hpp -- parameter layout of the decoder of include/rustral_model.h
// (the order its header documents), shared by the decoder and the serving
// engine.
#pragma once

#include <cstdint>

#include "../../include/rustral_model.h"

namespace rkv {

inline bool config_ok(const rkv_decoder_config* c) {
  if (!c || c->vocab <= 0 || c->d_model <= 0 || c->n_heads <= 0 || c->n_kv_heads <= 0 ||
      c->d_ff <= 0 || c->n_layers <= 0 || c->max_seq <= 0)
    return false;
  return c->d_model % c->n_heads == 0 && c->n_heads % c->n_kv_heads == 0;
}

struct LayerOffsets {
  int64_t ln1_g, ln1_b, wq, bq, wk, bk, wv, bv, wo, bo, ln2_g, ln2_b, w1, b1, w2, b2, end;
};

// Offsets of layer l's parameters (and the final norm / lm_head after them).
inline LayerOffsets layer_offsets(const rkv_decoder_config& c, int l) {
  const int64_t d = c.d_model, V = c.vocab, f = c.d_ff;
  const int64_t kvd = (int64_t)c.n_kv_heads * (d / c.n_heads);
  const int64_t per = 2 * d + (d * d + d) + 2 * (kvd * d + kvd) + (d * d + d) + 2 * d + (f * d + f) +
                      (d * f + d);
  LayerOffsets o;
  int64_t p = V * d + per * l;
  o.ln1_g = p; o.ln1_b = p + d; p += 2 * d;
  o.wq = p; o.bq = p + d * d; p += d * d + d;
  o.wk = p; o.bk = p + kvd * d; p += kvd * d + kvd;
  o.wv = p; o.bv = p + kvd * d; p += kvd * d + kvd;
  o.wo = p; o.bo = p + d * d; p += d * d + d;
  o.ln2_g = p; o.ln2_b = p + d; p += 2 * d;
  o.w1 = p; o.b1 = p + f * d; p += f * d + f;
  o.w2 = p; o.b2 = p + d * f; p += d * f + d;
  o.end = p;
  return o;
}

inline int64_t param_count(const rkv_decoder_config& c) {
  const int64_t d = c.d_model, V = c.vocab;
  return layer_offsets(c, c.n_layers - 1).end + 2 * d + V * d;
}

}  // namespace rkv
