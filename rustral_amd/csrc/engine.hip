// engine.hip -- continuous-batching serving engine (include/rustral_model.h):
// the scheduler of rustral_serving.h decides each step's batch and the
// decoder runs over it on the device, all through this library's entry
// points.
//
// One step:
//   1. rkv_sched_schedule -> the batch: per request its input tokens (the
//      prompt -- or prompt + generated after a preemption -- while in
//      prefill, else the last generated token), the position of the first
//      input, its sequence length and block table.
//   2. host: the position and the pool slot of every input token.
//   3. device, all input tokens as rows: embed + positional table; per layer
//      pre-LN, Q/K/V projections, rkv_append of K/V into the layer's pool,
//      ONE rkv_prefill_attention call for the whole batch (a prefill row
//      attends causally, a decode row is the single-token case), output
//      projection + residual, pre-LN MLP + residual; then each request's last
//      row through the final norm, lm_head and rkv_argmax.
//   4. the tokens go back to the host and into rkv_sched_update.
// The reference's ServingEngine::step (crates/nn/src/continuous_batching.rs:
// 516-528) emits a dummy token per request; this is the model forward it
// leaves out.
#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <new>
#include <vector>

#include "../../include/rustral_model.h"
#include "../../include/rustral_serving.h"
#include "model_layout.hpp"
#include "model_ops.hpp"

struct rkv_engine {
  rkv_decoder_config cfg{};
  hipStream_t stream = nullptr;
  int d_head = 0, kvd = 0;
  int64_t num_blocks = 0;
  rkv_scheduler* sched = nullptr;
  float* params = nullptr;  // device copy of the parameter array
  float* pe = nullptr;      // [max_seq][d] positional table
  float* k_pool = nullptr;  // [n_layers][num_blocks][Hkv][16][d_head]
  float* v_pool = nullptr;
  // per-step buffers, grown on demand: tokens (rows) and requests
  int64_t cap_tok = 0, cap_req = 0, cap_tab = 0;
  int32_t *ids = nullptr, *pos = nullptr, *q_start = nullptr, *ctx = nullptr, *tables = nullptr,
          *last = nullptr, *out_tok = nullptr;
  int64_t* slots = nullptr;
  float *x = nullptr, *q = nullptr, *o = nullptr, *f2 = nullptr, *xl = nullptr,
        *logits = nullptr;
};

namespace {

template <typename T>
bool dalloc(T*& p, size_t n) {
  return hipMalloc(reinterpret_cast<void**>(&p), n * sizeof(T)) == hipSuccess;
}

template <typename T>
void dfree(T*& p) {
  if (p) (void)hipFree(p);
  p = nullptr;
}

void free_step_buffers(rkv_engine* e) {
  dfree(e->ids), dfree(e->pos), dfree(e->q_start), dfree(e->ctx), dfree(e->tables);
  dfree(e->last), dfree(e->out_tok), dfree(e->slots);
  dfree(e->x), dfree(e->q), dfree(e->o);
  dfree(e->f2), dfree(e->xl), dfree(e->logits);
  e->cap_tok = e->cap_req = e->cap_tab = 0;
}

void release(rkv_engine* e) {
  if (!e) return;
  if (e->stream) (void)hipStreamSynchronize(e->stream);
  free_step_buffers(e);
  dfree(e->params), dfree(e->pe), dfree(e->k_pool), dfree(e->v_pool);
  if (e->sched) rkv_sched_destroy(e->sched);
  delete e;
}

// Makes the per-step buffers hold n_tok rows, n_req requests and n_req
// tables of mb blocks (doubling, so a run reallocates a few times at most).
bool reserve(rkv_engine* e, int64_t n_tok, int64_t n_req, int64_t mb) {
  if (n_tok <= e->cap_tok && n_req <= e->cap_req && n_req * mb <= e->cap_tab) return true;
  (void)hipStreamSynchronize(e->stream);  // the old buffers may still be read
  const int64_t ct = std::max(n_tok, 2 * e->cap_tok), cr = std::max(n_req, 2 * e->cap_req);
  const int64_t cb = std::max(n_req * mb, 2 * e->cap_tab);
  free_step_buffers(e);
  const rkv_decoder_config& c = e->cfg;
  const size_t d = (size_t)c.d_model, f = (size_t)c.d_ff;
  const bool ok = dalloc(e->ids, ct) && dalloc(e->pos, ct) && dalloc(e->slots, ct) &&
                  dalloc(e->q_start, cr + 1) && dalloc(e->ctx, cr) && dalloc(e->last, cr) &&
                  dalloc(e->out_tok, cr) && dalloc(e->tables, cb) && dalloc(e->x, ct * d) &&
                  dalloc(e->q, ct * d) && dalloc(e->o, ct * d) && dalloc(e->f2, ct * f) &&
                  dalloc(e->xl, cr * d) && dalloc(e->logits, cr * (size_t)c.vocab);
  if (!ok) {
    free_step_buffers(e);
    return false;
  }
  e->cap_tok = ct, e->cap_req = cr, e->cap_tab = cb;
  return true;
}

#define RKV_TRY(expr)              \
  do {                             \
    const int rc_ = (expr);        \
    if (rc_ != RKV_OK) return rc_; \
  } while (0)

}  // namespace

using namespace rkv;

extern "C" rkv_engine* rkv_engine_create(const rkv_decoder_config* cfg, const float* host_params,
                                         int64_t n_params, int64_t num_blocks, int max_batch_size,
                                         void* stream) {
  clear_error();
  if (!config_ok(cfg) || !host_params || num_blocks < 1 || max_batch_size < 1) {
    set_error("rkv_engine_create: bad configuration, parameters or sizes");
    return nullptr;
  }
  const rkv_decoder_config c = *cfg;
  const int dh = c.d_model / c.n_heads;
  if ((dh != 32 && dh != 64 && dh != 128) || (c.n_heads / c.n_kv_heads > 8)) {
    set_error("rkv_engine_create: head_dim must be 32, 64 or 128 and n_heads/n_kv_heads <= 8");
    return nullptr;
  }
  if (n_params != param_count(c)) {
    set_error("rkv_engine_create: n_params does not match rkv_decoder_param_count");
    return nullptr;
  }
  auto* e = new (std::nothrow) rkv_engine;
  if (!e) return nullptr;
  e->cfg = c;
  e->stream = static_cast<hipStream_t>(stream);
  e->d_head = dh;
  e->kvd = c.n_kv_heads * dh;
  e->num_blocks = num_blocks;
  const size_t d = (size_t)c.d_model, S = (size_t)c.max_seq;
  const size_t pool = (size_t)c.n_layers * (size_t)num_blocks * 16 * (size_t)e->kvd;
  bool ok = dalloc(e->params, (size_t)n_params) && dalloc(e->pe, S * d) &&
            dalloc(e->k_pool, pool) && dalloc(e->v_pool, pool);
  std::vector<float> pe(S * d);  // the reference's fp32 sinusoid (transformer.rs:69-82)
  for (size_t p = 0; p < S; ++p)
    for (size_t i = 0; i < d; ++i) {
      const float angle = (float)p / std::pow(10000.0f, (float)(2 * (i / 2)) / (float)d);
      pe[p * d + i] = (i % 2 == 0) ? std::sin(angle) : std::cos(angle);
    }
  ok = ok &&
       hipMemcpyAsync(e->params, host_params, (size_t)n_params * sizeof(float),
                      hipMemcpyHostToDevice, e->stream) == hipSuccess &&
       hipMemcpyAsync(e->pe, pe.data(), pe.size() * sizeof(float), hipMemcpyHostToDevice,
                      e->stream) == hipSuccess &&
       hipStreamSynchronize(e->stream) == hipSuccess;
  e->sched = ok ? rkv_sched_create(num_blocks, 16, max_batch_size, c.max_seq) : nullptr;
  if (!ok || !e->sched) {
    set_error("rkv_engine_create: device allocation, upload or scheduler setup failed");
    release(e);
    return nullptr;
  }
  return e;
}

extern "C" void rkv_engine_destroy(rkv_engine* e) { release(e); }

extern "C" rkv_scheduler* rkv_engine_scheduler(rkv_engine* e) { return e ? e->sched : nullptr; }

extern "C" int64_t rkv_engine_submit(rkv_engine* e, const int32_t* prompt, int n_prompt,
                                     int max_tokens, int priority) {
  clear_error();
  if (!e || !prompt || n_prompt < 1)
    return fail(RKV_ERR_INVALID_ARG, "rkv_engine_submit: bad argument");
  for (int i = 0; i < n_prompt; ++i)
    if (prompt[i] < 0 || prompt[i] >= e->cfg.vocab)
      return fail(RKV_ERR_INVALID_ARG, "rkv_engine_submit: prompt id outside [0, vocab)");
  return rkv_sched_add_request(e->sched, prompt, n_prompt, max_tokens, priority);
}

extern "C" int rkv_engine_step(rkv_engine* e) {
  clear_error();
  if (!e) return fail(RKV_ERR_INVALID_ARG, "rkv_engine_step: null engine");
  const int n = rkv_sched_schedule(e->sched);
  if (n <= 0) return n;
  int n_req = 0, mb = 0;
  int64_t n_tok = 0;
  RKV_TRY(rkv_sched_batch_dims(e->sched, &n_req, &n_tok, &mb));
  std::vector<int64_t> req((size_t)n_req), off((size_t)n_req + 1), slots((size_t)n_tok);
  std::vector<int32_t> lens((size_t)n_req), in_ids((size_t)n_tok), first((size_t)n_req),
      tab((size_t)n_req * mb), tok_pos((size_t)n_tok), q_start((size_t)n_req + 1),
      last((size_t)n_req);
  RKV_TRY(rkv_sched_batch(e->sched, req.data(), lens.data(), off.data(), in_ids.data(),
                          first.data(), tab.data(), mb));
  const rkv_decoder_config& c = e->cfg;
  int max_q = 0;
  for (int r = 0; r < n_req; ++r) {
    const int64_t n_in = off[(size_t)r + 1] - off[(size_t)r];
    max_q = std::max(max_q, (int)n_in);
    q_start[(size_t)r] = (int32_t)off[(size_t)r];
    last[(size_t)r] = (int32_t)(off[(size_t)r + 1] - 1);
    for (int64_t i = 0; i < n_in; ++i) {
      const int64_t t = off[(size_t)r] + i;
      const int p = first[(size_t)r] + (int)i;
      if (p >= c.max_seq) return fail(RKV_ERR_INVALID_ARG, "rkv_engine_step: position >= max_seq");
      tok_pos[(size_t)t] = p;
      // the scheduler hands out tables that cover every row's sequence; a
      // position past the row's table is refused rather than read out of it
      const int32_t blk = p / 16 < mb ? tab[(size_t)r * mb + p / 16] : -1;
      if (blk < 0 || blk >= e->num_blocks)
        return fail(RKV_ERR_OOM, "rkv_engine_step: position without a block (KV cache out of memory)");
      slots[(size_t)t] = (int64_t)blk * 16 + p % 16;
    }
  }
  q_start[(size_t)n_req] = (int32_t)off[(size_t)n_req];
  if (!reserve(e, n_tok, n_req, mb))
    return fail(RKV_ERR_HIP, "rkv_engine_step: device allocation failed");
  hipStream_t s = e->stream;
  auto up = [&](void* dst, const void* src, size_t bytes) {
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s) == hipSuccess;
  };
  if (!up(e->ids, in_ids.data(), in_ids.size() * 4) || !up(e->pos, tok_pos.data(), tok_pos.size() * 4) ||
      !up(e->slots, slots.data(), slots.size() * 8) ||
      !up(e->q_start, q_start.data(), q_start.size() * 4) ||
      !up(e->ctx, lens.data(), lens.size() * 4) || !up(e->tables, tab.data(), tab.size() * 4) ||
      !up(e->last, last.data(), last.size() * 4))
    return fail(RKV_ERR_HIP, "rkv_engine_step: upload failed");

  const int d = c.d_model, f = c.d_ff, V = c.vocab, H = c.n_heads, Hk = c.n_kv_heads;
  const int dh = e->d_head, T = (int)n_tok;
  const float scale = 1.0f / std::sqrt((float)dh);  // tape_transformer.rs:75
  const int64_t layer_pool = e->num_blocks * Hk * 16 * dh;
  const float* P = e->params;
  RKV_TRY(rkv_embed(e->x, P, e->ids, e->pe, e->pos, T, V, d, c.max_seq, s));
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerOffsets o = layer_offsets(c, l);
    float* kp = e->k_pool + l * layer_pool;
    float* vp = e->v_pool + l * layer_pool;
    // LN1, q / k / v projections and the KV append in one launch
    RKV_TRY(rkv_qkv_append(e->q, kp, vp, e->slots, e->x, P + o.ln1_g, P + o.ln1_b, c.eps,
                           P + o.wq, P + o.bq, P + o.wk, P + o.bk, P + o.wv, P + o.bv, T, d, d,
                           Hk, dh, 16, e->num_blocks, RKV_F32, s));
    RKV_TRY(rkv_prefill_attention(e->o, e->q, kp, vp, e->tables, mb, e->q_start, e->ctx, n_req,
                                  H, Hk, dh, 16, e->num_blocks, max_q, scale, RKV_F32, s));
    // x += o W_o^T + b_o; x += gelu(LN2(x) W_1^T + b_1) W_2^T + b_2 (fused epilogues)
    RKV_TRY(linear_launch(e->x, e->o, P + o.wo, P + o.bo, e->x, 1, T, d, d, s));
    RKV_TRY(linear_launch(e->f2, e->x, P + o.w1, P + o.b1, nullptr, 2, T, d, f, s, P + o.ln2_g,
                          P + o.ln2_b, c.eps));
    RKV_TRY(linear_launch(e->x, e->f2, P + o.w2, P + o.b2, e->x, 1, T, f, d, s));
  }
  // each request's last row: final norm, lm_head (no bias, transformer.rs:789), greedy
  const int64_t fin = layer_offsets(c, c.n_layers - 1).end;
  RKV_TRY(rkv_embed(e->xl, e->x, e->last, nullptr, nullptr, n_req, T, d, 0, s));
  RKV_TRY(linear_launch(e->logits, e->xl, P + fin + 2 * d, nullptr, nullptr, 0, n_req, d, V, s,
                        P + fin, P + fin + d, c.eps));
  RKV_TRY(rkv_argmax(e->out_tok, e->logits, n_req, V, s));
  std::vector<int32_t> tokens((size_t)n_req);
  if (hipMemcpyAsync(tokens.data(), e->out_tok, tokens.size() * 4, hipMemcpyDeviceToHost, s) !=
          hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return fail(RKV_ERR_HIP, "rkv_engine_step: copy back failed");
  RKV_TRY(rkv_sched_update(e->sched, req.data(), tokens.data(), n_req));
  return n_req;
}

extern "C" int rkv_engine_run(rkv_engine* e, int max_steps) {
  clear_error();
  if (!e || max_steps < 0) return fail(RKV_ERR_INVALID_ARG, "rkv_engine_run: bad argument");
  int steps = 0;
  while (steps < max_steps) {
    const int n = rkv_engine_step(e);
    if (n < 0) return n;
    if (n == 0) break;
    ++steps;
  }
  return steps;
}
