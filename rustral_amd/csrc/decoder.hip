// decoder.hip -- host side of the greedy decoder (include/rustral_model.h):
// parameter upload, paged KV pools fed by the host block manager, and the
// per-token launch sequence over the library's own entry points.  Also the
// seeded PCG64 / Box-Muller generator used for random initialisation.
//
// A step keeps everything on the device: the token ids live in a device
// array (prompt ids uploaded once, generated ids written there by
// rkv_argmax), the slot of every position and the context length of every
// step are precomputed, so the stream is synchronized once per call.  The
// launch sequence depends only on the call's shape (prompt length, tokens to
// generate): it is captured once into a HIP graph and replayed by every
// later call of that shape, the per-call data (ids, block table, slots)
// uploaded into the same device buffers beforehand.
#include "common.hpp"

#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/rustral_model.h"
#include "../../include/rustral_serving.h"
#include "model_layout.hpp"
#include "model_ops.hpp"
#include "safetensors.hpp"

// ---- generator -------------------------------------------------------------------

namespace rkv {
namespace {

struct Pcg64 {
  unsigned __int128 state, inc;
  static unsigned __int128 mult() {
    return ((unsigned __int128)0x2360ED051FC65DA4ull << 64) | 0x4385DF649FCCF645ull;
  }
  explicit Pcg64(uint64_t seed)
      : state(seed), inc(((unsigned __int128)0xDA3E39CB94B95BDBull << 1) | 1u) {}
  uint64_t next() {
    state = state * mult() + inc;
    const uint64_t x = (uint64_t)(state >> 64) ^ (uint64_t)state;
    const unsigned rot = (unsigned)(state >> 122);
    return (x >> rot) | (x << ((64u - rot) & 63u));
  }
  double uniform() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }
};

void fill_normal(float* out, int64_t n, Pcg64& g, float std) {
  const double two_pi = 6.283185307179586476925286766559;
  for (int64_t i = 0; i < n; i += 2) {
    const double u1 = g.uniform(), u2 = g.uniform();
    const double r = std::sqrt(-2.0 * std::log(1.0 - u1));
    out[i] = (float)(std * (r * std::cos(two_pi * u2)));
    if (i + 1 < n) out[i + 1] = (float)(std * (r * std::sin(two_pi * u2)));
  }
}

}  // namespace
}  // namespace rkv

using namespace rkv;

extern "C" int rkv_rng_raw(uint64_t seed, uint64_t* out, int64_t n) {
  clear_error();
  if (n < 0 || (n > 0 && !out)) return fail(RKV_ERR_INVALID_ARG, "rkv_rng_raw: bad argument");
  Pcg64 g(seed);
  for (int64_t i = 0; i < n; ++i) out[i] = g.next();
  return RKV_OK;
}

extern "C" int rkv_fill_normal(float* out, int64_t n, uint64_t seed, float std) {
  clear_error();
  if (n < 0 || (n > 0 && !out)) return fail(RKV_ERR_INVALID_ARG, "rkv_fill_normal: bad argument");
  Pcg64 g(seed);
  fill_normal(out, n, g, std);
  return RKV_OK;
}

extern "C" int64_t rkv_decoder_param_count(const rkv_decoder_config* cfg) {
  if (!config_ok(cfg)) return -1;
  return param_count(*cfg);
}

extern "C" int rkv_decoder_init_params(const rkv_decoder_config* cfg, uint64_t seed, float std,
                                       float* host_params) {
  clear_error();
  if (!config_ok(cfg) || !host_params)
    return fail(RKV_ERR_INVALID_ARG, "rkv_decoder_init_params: bad argument");
  const rkv_decoder_config& c = *cfg;
  const int64_t d = c.d_model, V = c.vocab, f = c.d_ff;
  const int64_t kvd = (int64_t)c.n_kv_heads * (d / c.n_heads);
  Pcg64 g(seed);
  float* P = host_params;
  auto normal = [&](int64_t off, int64_t n) { fill_normal(P + off, n, g, std); };
  auto fill = [&](int64_t off, int64_t n, float v) {
    for (int64_t i = 0; i < n; ++i) P[off + i] = v;
  };
  normal(0, V * d);
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerOffsets o = layer_offsets(c, l);
    fill(o.ln1_g, d, 1.0f); fill(o.ln1_b, d, 0.0f);
    normal(o.wq, d * d); fill(o.bq, d, 0.0f);
    normal(o.wk, kvd * d); fill(o.bk, kvd, 0.0f);
    normal(o.wv, kvd * d); fill(o.bv, kvd, 0.0f);
    normal(o.wo, d * d); fill(o.bo, d, 0.0f);
    fill(o.ln2_g, d, 1.0f); fill(o.ln2_b, d, 0.0f);
    normal(o.w1, f * d); fill(o.b1, f, 0.0f);
    normal(o.w2, d * f); fill(o.b2, d, 0.0f);
  }
  const int64_t fin = layer_offsets(c, c.n_layers - 1).end;
  fill(fin, d, 1.0f);
  fill(fin + d, d, 0.0f);
  normal(fin + 2 * d, V * d);
  return RKV_OK;
}

// ---- decoder ----------------------------------------------------------------------

struct rkv_decoder {
  rkv_decoder_config cfg{};
  hipStream_t stream = nullptr;
  hipStream_t own_stream = nullptr;  // created when the caller passes no stream
  hipGraphExec_t graph = nullptr;    // the launch sequence of the last shape
  int graph_prompt = -1, graph_total = -1;
  int d_head = 0, kvd = 0, num_blocks = 0;
  float* params = nullptr;   // device copy of the parameter array
  float* pe = nullptr;       // [max_seq][d] positional table
  float* k_pool = nullptr;   // [n_layers][num_blocks][Hkv][16][d_head]
  float* v_pool = nullptr;
  int32_t* ids = nullptr;    // [max_seq + 1] token ids by position
  int32_t* pos = nullptr;    // [max_seq] position p at index p
  int32_t* ctx = nullptr;    // [max_seq] context length p + 1 at index p
  int64_t* slots = nullptr;  // [max_seq] pool slot of position p
  int32_t* table = nullptr;  // [max_blocks] block table of the sequence
  float* logits = nullptr;   // [max_seq][vocab]
  float *x = nullptr, *q = nullptr, *o = nullptr, *f2 = nullptr;
  void* ws = nullptr;
  size_t ws_bytes = 0;
  rkv_block_manager* bm = nullptr;
};

namespace {

template <typename T>
bool dalloc(T*& p, size_t n) {
  return hipMalloc(reinterpret_cast<void**>(&p), n * sizeof(T)) == hipSuccess;
}

void release(rkv_decoder* dec) {
  if (!dec) return;
  void* bufs[] = {dec->params, dec->pe,  dec->k_pool, dec->v_pool, dec->ids,   dec->pos,
                  dec->ctx,    dec->slots, dec->table, dec->logits, dec->x,     dec->q,
                  dec->o,      dec->f2,  dec->ws};
  if (dec->graph) (void)hipGraphExecDestroy(dec->graph);
  for (void* b : bufs)
    if (b) (void)hipFree(b);
  if (dec->bm) rkv_bm_destroy(dec->bm);
  if (dec->own_stream) (void)hipStreamDestroy(dec->own_stream);
  delete dec;
}

#define RKV_TRY(expr)             \
  do {                            \
    const int rc_ = (expr);       \
    if (rc_ != RKV_OK) return rc_; \
  } while (0)

}  // namespace

extern "C" void rkv_decoder_destroy(rkv_decoder* dec) { release(dec); }

namespace rkv {
int copy_tensors(const st::File& f, const std::vector<const st::Tensor*>& found,
                 const std::vector<void*>& dsts, bool on_device, hipStream_t stream,
                 const char* what);
}  // namespace rkv

namespace {
// Allocates a decoder; uploads host_params unless it is NULL (the caller then
// fills dec->params itself, as the safetensors loader does).
rkv_decoder* create(const rkv_decoder_config* cfg, const float* host_params, int64_t n_params,
                    void* stream);
}  // namespace

extern "C" rkv_decoder* rkv_decoder_create(const rkv_decoder_config* cfg, const float* host_params,
                                           int64_t n_params, void* stream) {
  clear_error();
  if (!config_ok(cfg) || !host_params) {
    set_error("rkv_decoder_create: bad configuration or null parameters");
    return nullptr;
  }
  return create(cfg, host_params, n_params, stream);
}

extern "C" int rkv_decoder_load_safetensors_device(rkv_decoder* dec, const char* path) {
  clear_error();
  if (!dec || !path) return fail(RKV_ERR_INVALID_ARG, "rkv_decoder_load_safetensors_device: bad argument");
  std::string err;
  std::unique_ptr<st::File> f = st::open(path, err);
  if (!f) return fail(RKV_ERR_INVALID_ARG, err);
  std::vector<int64_t> offsets;
  const std::vector<st::Want> want = st::decoder_layout(dec->cfg, &offsets);
  std::vector<const st::Tensor*> found;
  if (!st::match(*f, want, found, err)) return fail(RKV_ERR_INVALID_ARG, err);
  std::vector<void*> dst(want.size());
  for (size_t i = 0; i < want.size(); ++i) dst[i] = dec->params + offsets[i];
  return copy_tensors(*f, found, dst, true, dec->stream, "rkv_decoder_load_safetensors_device");
}

extern "C" rkv_decoder* rkv_decoder_create_from_safetensors(const rkv_decoder_config* cfg,
                                                            const char* path, void* stream) {
  clear_error();
  if (!config_ok(cfg) || !path) {
    set_error("rkv_decoder_create_from_safetensors: bad configuration or null path");
    return nullptr;
  }
  rkv_decoder* dec = create(cfg, nullptr, param_count(*cfg), stream);
  if (!dec) return nullptr;
  if (rkv_decoder_load_safetensors_device(dec, path) != RKV_OK) {
    const std::string msg = rkv_last_error();
    release(dec);
    set_error(msg);
    return nullptr;
  }
  return dec;
}

namespace {
rkv_decoder* create(const rkv_decoder_config* cfg, const float* host_params, int64_t n_params,
                    void* stream) {
  const rkv_decoder_config c = *cfg;
  const int dh = c.d_model / c.n_heads;
  if ((dh != 32 && dh != 64 && dh != 128) || (c.n_heads / c.n_kv_heads > 8)) {
    set_error("rkv_decoder_create: head_dim must be 32, 64 or 128 and n_heads/n_kv_heads <= 8");
    return nullptr;
  }
  if (n_params != param_count(c)) {
    set_error("rkv_decoder_create: n_params does not match rkv_decoder_param_count");
    return nullptr;
  }
  auto* dec = new (std::nothrow) rkv_decoder;
  if (!dec) return nullptr;
  dec->cfg = c;
  dec->stream = static_cast<hipStream_t>(stream);
  if (!dec->stream) {  // graph capture needs a stream of its own
    if (hipStreamCreateWithFlags(&dec->own_stream, hipStreamNonBlocking) != hipSuccess) {
      set_error("rkv_decoder_create: stream creation failed");
      release(dec);
      return nullptr;
    }
    dec->stream = dec->own_stream;
  }
  dec->d_head = dh;
  dec->kvd = c.n_kv_heads * dh;
  dec->num_blocks = (c.max_seq + 15) / 16;
  const size_t d = (size_t)c.d_model, S = (size_t)c.max_seq;
  const size_t pool = (size_t)c.n_layers * dec->num_blocks * 16 * dec->kvd;
  bool ok = dalloc(dec->params, (size_t)n_params) && dalloc(dec->pe, S * d) &&
            dalloc(dec->k_pool, pool) && dalloc(dec->v_pool, pool) && dalloc(dec->ids, S + 1) &&
            dalloc(dec->pos, S) && dalloc(dec->ctx, S) && dalloc(dec->slots, S) &&
            dalloc(dec->table, (size_t)dec->num_blocks) &&
            dalloc(dec->logits, S * (size_t)c.vocab) && dalloc(dec->x, d) && dalloc(dec->q, d) &&
            dalloc(dec->o, d) && dalloc(dec->f2, (size_t)c.d_ff);
  dec->ws_bytes = rkv_decode_workspace_bytes(1, c.n_heads, dh, c.max_seq, 0);
  if (ok && dec->ws_bytes) ok = hipMalloc(&dec->ws, dec->ws_bytes) == hipSuccess;
  if (!ok) {
    set_error("rkv_decoder_create: device allocation failed");
    release(dec);
    return nullptr;
  }
  // positional table: same fp32 formula as the reference (transformer.rs:69-82)
  std::vector<float> pe(S * d);
  for (size_t p = 0; p < S; ++p)
    for (size_t i = 0; i < d; ++i) {
      const float angle = (float)p / std::pow(10000.0f, (float)(2 * (i / 2)) / (float)d);
      pe[p * d + i] = (i % 2 == 0) ? std::sin(angle) : std::cos(angle);
    }
  std::vector<int32_t> pos(S), ctx(S);
  for (size_t p = 0; p < S; ++p) {
    pos[p] = (int32_t)p;
    ctx[p] = (int32_t)(p + 1);
  }
  hipStream_t s = dec->stream;
  ok = (!host_params || hipMemcpyAsync(dec->params, host_params, (size_t)n_params * sizeof(float),
                                       hipMemcpyHostToDevice, s) == hipSuccess) &&
       hipMemcpyAsync(dec->pe, pe.data(), pe.size() * sizeof(float), hipMemcpyHostToDevice, s) ==
           hipSuccess &&
       hipMemcpyAsync(dec->pos, pos.data(), S * sizeof(int32_t), hipMemcpyHostToDevice, s) ==
           hipSuccess &&
       hipMemcpyAsync(dec->ctx, ctx.data(), S * sizeof(int32_t), hipMemcpyHostToDevice, s) ==
           hipSuccess &&
       hipStreamSynchronize(s) == hipSuccess;
  dec->bm = rkv_bm_create(dec->num_blocks, 16);
  if (!ok || !dec->bm) {
    set_error("rkv_decoder_create: upload or block manager setup failed");
    release(dec);
    return nullptr;
  }
  return dec;
}
}  // namespace

namespace {

// Enqueues the launch sequence of one generation on s: positions 0 ..
// total - 1, logits and the greedy id for every position from n_prompt - 1
// on.  Everything it reads per call (ids, block table, slots) comes from the
// decoder's device buffers, so the sequence depends only on the shape.
int enqueue_generation(rkv_decoder* dec, int n_prompt, int total, hipStream_t s) {
  const rkv_decoder_config& c = dec->cfg;
  const int d = c.d_model, f = c.d_ff, V = c.vocab, H = c.n_heads, Hk = c.n_kv_heads;
  const int dh = dec->d_head;
  const float scale = 1.0f / std::sqrt((float)dh);  // tape_transformer.rs:75
  const int64_t layer_pool = (int64_t)dec->num_blocks * Hk * 16 * dh;
  const float* P = dec->params;
  const int64_t fin = layer_offsets(c, c.n_layers - 1).end;
  int produced = 0;
  for (int p = 0; p < total; ++p) {
    RKV_TRY(rkv_embed(dec->x, P, dec->ids + p, dec->pe, dec->pos + p, 1, V, d, c.max_seq, s));
    for (int l = 0; l < c.n_layers; ++l) {
      const LayerOffsets o = layer_offsets(c, l);
      float* kp = dec->k_pool + l * layer_pool;
      float* vp = dec->v_pool + l * layer_pool;
      // LN1, q / k / v projections and the KV append in one launch
      RKV_TRY(rkv_qkv_append(dec->q, kp, vp, dec->slots + p, dec->x, P + o.ln1_g, P + o.ln1_b,
                             c.eps, P + o.wq, P + o.bq, P + o.wk, P + o.bk, P + o.wv, P + o.bv, 1,
                             d, d, Hk, dh, 16, dec->num_blocks, RKV_F32, s));
      RKV_TRY(rkv_decode_attention(dec->o, dec->q, kp, vp, dec->table, dec->num_blocks,
                                   dec->ctx + p, 1, H, Hk, dh, 16, dec->num_blocks, c.max_seq,
                                   scale, RKV_F32, 0, dec->ws, dec->ws_bytes, s));
      // x += o W_o^T + b_o; x += gelu(LN2(x) W_1^T + b_1) W_2^T + b_2 (fused epilogues)
      RKV_TRY(linear_launch(dec->x, dec->o, P + o.wo, P + o.bo, dec->x, 1, 1, d, d, s));
      RKV_TRY(linear_launch(dec->f2, dec->x, P + o.w1, P + o.b1, nullptr, 2, 1, d, f, s,
                            P + o.ln2_g, P + o.ln2_b, c.eps));
      RKV_TRY(linear_launch(dec->x, dec->f2, P + o.w2, P + o.b2, dec->x, 1, 1, f, d, s));
    }
    if (p + 1 < n_prompt) continue;  // prompt ids are known
    float* lg = dec->logits + (int64_t)produced * V;
    RKV_TRY(linear_launch(lg, dec->x, P + fin + 2 * d, nullptr, nullptr, 0, 1, d, V, s, P + fin,
                          P + fin + d, c.eps));
    RKV_TRY(rkv_argmax(dec->ids + p + 1, lg, 1, V, s));
    ++produced;
  }
  return RKV_OK;
}

// Captures enqueue_generation for this shape into dec->graph (replacing the
// previous shape's graph).
int capture_generation(rkv_decoder* dec, int n_prompt, int total) {
  hipStream_t s = dec->stream;
  if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess)
    return fail(RKV_ERR_HIP, "rkv_decoder_generate: stream capture failed to start");
  const int rc = enqueue_generation(dec, n_prompt, total, s);
  hipGraph_t g = nullptr;
  const hipError_t ec = hipStreamEndCapture(s, &g);
  if (rc != RKV_OK) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (ec != hipSuccess || !g) return fail(RKV_ERR_HIP, "rkv_decoder_generate: stream capture failed");
  hipGraphExec_t x = nullptr;
  const hipError_t ei = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (ei != hipSuccess) return fail(RKV_ERR_HIP, "rkv_decoder_generate: graph instantiation failed");
  if (dec->graph) (void)hipGraphExecDestroy(dec->graph);
  dec->graph = x;
  dec->graph_prompt = n_prompt;
  dec->graph_total = total;
  return RKV_OK;
}

}  // namespace

extern "C" int rkv_decoder_generate(rkv_decoder* dec, const int32_t* prompt, int n_prompt,
                                    int n_new, int32_t* out_tokens, float* out_logits) {
  clear_error();
  if (!dec || !prompt || n_prompt < 1 || n_new < 0 || (n_new > 0 && !out_tokens))
    return fail(RKV_ERR_INVALID_ARG, "rkv_decoder_generate: bad argument");
  const rkv_decoder_config& c = dec->cfg;
  const int total = n_prompt + (n_new > 0 ? n_new - 1 : 0);
  if (total > c.max_seq)
    return fail(RKV_ERR_INVALID_ARG, "rkv_decoder_generate: prompt + new tokens exceed max_seq");
  for (int i = 0; i < n_prompt; ++i)
    if (prompt[i] < 0 || prompt[i] >= c.vocab)
      return fail(RKV_ERR_INVALID_ARG, "rkv_decoder_generate: prompt id outside [0, vocab)");
  if (n_new == 0) return RKV_OK;
  hipStream_t s = dec->stream;

  // Blocks for the whole generation from the block manager (sequence 0), in
  // the order a growing sequence takes them; the slot of position p is
  // table[p / 16] * 16 + p % 16.
  rkv_bm_free(dec->bm, 0);
  if (rkv_bm_reserve(dec->bm, 0, total) < 0)
    return fail(RKV_ERR_OOM, "rkv_decoder_generate: KV pool exhausted");
  std::vector<int32_t> table((size_t)dec->num_blocks, -1);
  const int64_t nb = rkv_bm_table(dec->bm, 0, table.data(), dec->num_blocks);
  std::vector<int64_t> slots((size_t)total);
  for (int p = 0; p < total; ++p) slots[(size_t)p] = (int64_t)table[(size_t)(p / 16)] * 16 + p % 16;
  if (hipMemcpyAsync(dec->table, table.data(), table.size() * sizeof(int32_t),
                     hipMemcpyHostToDevice, s) != hipSuccess ||
      hipMemcpyAsync(dec->slots, slots.data(), slots.size() * sizeof(int64_t),
                     hipMemcpyHostToDevice, s) != hipSuccess ||
      hipMemcpyAsync(dec->ids, prompt, (size_t)n_prompt * sizeof(int32_t), hipMemcpyHostToDevice,
                     s) != hipSuccess)
    return fail(RKV_ERR_HIP, "rkv_decoder_generate: upload failed");
  (void)nb;

  if (!dec->graph || dec->graph_prompt != n_prompt || dec->graph_total != total)
    RKV_TRY(capture_generation(dec, n_prompt, total));
  if (hipGraphLaunch(dec->graph, s) != hipSuccess)
    return fail(RKV_ERR_HIP, "rkv_decoder_generate: graph launch failed");
  if (hipMemcpyAsync(out_tokens, dec->ids + n_prompt, (size_t)n_new * sizeof(int32_t),
                     hipMemcpyDeviceToHost, s) != hipSuccess ||
      (out_logits && hipMemcpyAsync(out_logits, dec->logits, (size_t)n_new * c.vocab * sizeof(float),
                                    hipMemcpyDeviceToHost, s) != hipSuccess) ||
      hipStreamSynchronize(s) != hipSuccess)
    return fail(RKV_ERR_HIP, "rkv_decoder_generate: copy back failed");
  return RKV_OK;
}
