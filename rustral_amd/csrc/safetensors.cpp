// safetensors.cpp -- the decoder's parameters in the safetensors format
// (include/rustral_model.h): a strict loader into the packed parameter array
// and the matching writer.  Host code only.
//
// File format: 8-byte little-endian header length N, N bytes of JSON
// {"<name>": {"dtype": "F32", "shape": [..], "data_offsets": [begin, end]},
//  ..., "__metadata__": {"<key>": "<value>"}}, then the data bytes; offsets
// are relative to the end of the header.
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/rustral_kv.h"
#include "../../include/rustral_model.h"
#include "model_layout.hpp"

namespace rkv {
void set_error(const std::string& msg);
void clear_error();
}  // namespace rkv

namespace {

using rkv::set_error;

int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

// ---- a small JSON reader for the header ------------------------------------

struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  double num = 0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;
};

struct Parser {
  const char* p;
  const char* end;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if ((size_t)(end - p) < n || std::strncmp(p, s, n) != 0) return false;
    p += n;
    return true;
  }
  bool string(std::string& out) {
    if (p >= end || *p != '"') return false;
    ++p;
    while (p < end && *p != '"') {
      char c = *p++;
      if (c == '\\') {
        if (p >= end) return false;
        c = *p++;
        switch (c) {
          case '"': case '\\': case '/': out += c; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {  // \uXXXX, encoded as UTF-8 (no surrogate pairs: not in tensor names)
            if (end - p < 4) return false;
            unsigned v = 0;
            for (int i = 0; i < 4; ++i) {
              const char h = *p++;
              v = v * 16 + (h >= '0' && h <= '9' ? h - '0'
                            : h >= 'a' && h <= 'f' ? h - 'a' + 10
                            : h >= 'A' && h <= 'F' ? h - 'A' + 10 : 99);
              if (v > 0xffff) return false;
            }
            if (v < 0x80) {
              out += (char)v;
            } else if (v < 0x800) {
              out += (char)(0xc0 | (v >> 6));
              out += (char)(0x80 | (v & 0x3f));
            } else {
              out += (char)(0xe0 | (v >> 12));
              out += (char)(0x80 | ((v >> 6) & 0x3f));
              out += (char)(0x80 | (v & 0x3f));
            }
            break;
          }
          default: return false;
        }
      } else {
        out += c;
      }
    }
    if (p >= end) return false;
    ++p;
    return true;
  }
  bool value(Json& v, int depth) {
    if (depth > 16) return false;
    ws();
    if (p >= end) return false;
    if (*p == '{') {
      ++p;
      v.kind = Json::Obj;
      ws();
      if (p < end && *p == '}') return ++p, true;
      for (;;) {
        ws();
        std::string k;
        if (!string(k)) return false;
        ws();
        if (p >= end || *p != ':') return false;
        ++p;
        Json x;
        if (!value(x, depth + 1)) return false;
        v.obj.emplace_back(std::move(k), std::move(x));
        ws();
        if (p < end && *p == ',') { ++p; continue; }
        if (p < end && *p == '}') return ++p, true;
        return false;
      }
    }
    if (*p == '[') {
      ++p;
      v.kind = Json::Arr;
      ws();
      if (p < end && *p == ']') return ++p, true;
      for (;;) {
        Json x;
        if (!value(x, depth + 1)) return false;
        v.arr.push_back(std::move(x));
        ws();
        if (p < end && *p == ',') { ++p; continue; }
        if (p < end && *p == ']') return ++p, true;
        return false;
      }
    }
    if (*p == '"') {
      v.kind = Json::Str;
      return string(v.str);
    }
    if (lit("true")) return v.kind = Json::Bool, v.num = 1, true;
    if (lit("false")) return v.kind = Json::Bool, v.num = 0, true;
    if (lit("null")) return v.kind = Json::Null, true;
    // number (tensor shapes and offsets are non-negative integers)
    const char* s = p;
    while (p < end && (*p == '-' || *p == '+' || *p == '.' || *p == 'e' || *p == 'E' ||
                       (*p >= '0' && *p <= '9')))
      ++p;
    if (p == s) return false;
    v.kind = Json::Num;
    v.num = std::strtod(std::string(s, p).c_str(), nullptr);
    return true;
  }
};

// ---- the decoder's names and shapes, in parameter order ---------------------

struct Entry {
  std::string name;
  std::vector<int64_t> shape;
  int64_t offset;  // into the packed parameter array (floats)
};

std::vector<Entry> layout(const rkv_decoder_config& c) {
  const int64_t d = c.d_model, V = c.vocab, f = c.d_ff;
  const int64_t kvd = (int64_t)c.n_kv_heads * (d / c.n_heads);
  std::vector<Entry> e;
  e.push_back({"token_embedding.weight", {V, d}, 0});
  for (int l = 0; l < c.n_layers; ++l) {
    const rkv::LayerOffsets o = rkv::layer_offsets(c, l);
    const std::string p = "layers." + std::to_string(l) + ".";
    e.push_back({p + "norm1.weight", {d}, o.ln1_g});
    e.push_back({p + "norm1.bias", {d}, o.ln1_b});
    e.push_back({p + "self_attn.q_proj.weight", {d, d}, o.wq});
    e.push_back({p + "self_attn.q_proj.bias", {d}, o.bq});
    e.push_back({p + "self_attn.k_proj.weight", {kvd, d}, o.wk});
    e.push_back({p + "self_attn.k_proj.bias", {kvd}, o.bk});
    e.push_back({p + "self_attn.v_proj.weight", {kvd, d}, o.wv});
    e.push_back({p + "self_attn.v_proj.bias", {kvd}, o.bv});
    e.push_back({p + "self_attn.out_proj.weight", {d, d}, o.wo});
    e.push_back({p + "self_attn.out_proj.bias", {d}, o.bo});
    e.push_back({p + "norm2.weight", {d}, o.ln2_g});
    e.push_back({p + "norm2.bias", {d}, o.ln2_b});
    e.push_back({p + "ff_linear1.weight", {f, d}, o.w1});
    e.push_back({p + "ff_linear1.bias", {f}, o.b1});
    e.push_back({p + "ff_linear2.weight", {d, f}, o.w2});
    e.push_back({p + "ff_linear2.bias", {d}, o.b2});
  }
  const int64_t fin = rkv::layer_offsets(c, c.n_layers - 1).end;
  e.push_back({"final_norm.weight", {d}, fin});
  e.push_back({"final_norm.bias", {d}, fin + d});
  e.push_back({"lm_head.weight", {V, d}, fin + 2 * d});
  return e;
}

std::string shape_str(const std::vector<int64_t>& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

std::string json_escape(const std::string& s) {
  std::string r;
  for (char ch : s) {
    if (ch == '"' || ch == '\\') r += '\\';
    r += ch;
  }
  return r;
}

bool read_file(const char* path, std::vector<uint8_t>& out, std::string& err) {
  FILE* f = std::fopen(path, "rb");
  if (!f) {
    err = std::string("cannot open ") + path + ": " + std::strerror(errno);
    return false;
  }
  uint8_t buf[1 << 16];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) out.insert(out.end(), buf, buf + n);
  const bool ok = !std::ferror(f);
  std::fclose(f);
  if (!ok) err = std::string("read error on ") + path;
  return ok;
}

}  // namespace

extern "C" int rkv_decoder_load_safetensors(const rkv_decoder_config* cfg, const char* path,
                                            float* host_params, int64_t n_params) {
  rkv::clear_error();
  if (!rkv::config_ok(cfg) || !path || !host_params)
    return fail(RKV_ERR_INVALID_ARG, "rkv_decoder_load_safetensors: bad argument");
  if (n_params != rkv::param_count(*cfg))
    return fail(RKV_ERR_INVALID_ARG,
                "rkv_decoder_load_safetensors: n_params does not match rkv_decoder_param_count");
  std::vector<uint8_t> data;
  std::string err;
  if (!read_file(path, data, err)) return fail(RKV_ERR_INVALID_ARG, err);
  if (data.size() < 8) return fail(RKV_ERR_INVALID_ARG, "safetensors: file shorter than 8 bytes");
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | data[(size_t)i];
  if (hlen > data.size() - 8) return fail(RKV_ERR_INVALID_ARG, "safetensors: header past the end");
  Parser ps{reinterpret_cast<const char*>(data.data()) + 8,
            reinterpret_cast<const char*>(data.data()) + 8 + hlen};
  Json root;
  if (!ps.value(root, 0) || root.kind != Json::Obj)
    return fail(RKV_ERR_INVALID_ARG, "safetensors: header is not a JSON object");
  const uint8_t* body = data.data() + 8 + hlen;
  const uint64_t body_len = data.size() - 8 - hlen;

  std::map<std::string, const Json*> tensors;
  for (const auto& kv : root.obj)
    if (kv.first != "__metadata__") tensors[kv.first] = &kv.second;
  const std::vector<Entry> want = layout(*cfg);
  // strict checks, as load_model (crates/runtime/src/model_io.rs:36-105)
  std::string missing, extra;
  for (const Entry& e : want)
    if (!tensors.count(e.name)) missing += (missing.empty() ? "" : ", ") + e.name;
  if (!missing.empty())
    return fail(RKV_ERR_INVALID_ARG, "load_model: missing keys: " + missing);
  for (const auto& kv : tensors) {
    bool known = false;
    for (const Entry& e : want) known = known || e.name == kv.first;
    if (!known) extra += (extra.empty() ? "" : ", ") + kv.first;
  }
  if (!extra.empty())
    return fail(RKV_ERR_INVALID_ARG, "load_model: unexpected extra keys: " + extra);
  for (const Entry& e : want) {
    const Json& t = *tensors[e.name];
    const Json *dt = nullptr, *sh = nullptr, *off = nullptr;
    if (t.kind == Json::Obj)
      for (const auto& kv : t.obj) {
        if (kv.first == "dtype") dt = &kv.second;
        if (kv.first == "shape") sh = &kv.second;
        if (kv.first == "data_offsets") off = &kv.second;
      }
    if (!dt || !sh || !off || dt->kind != Json::Str || sh->kind != Json::Arr ||
        off->kind != Json::Arr || off->arr.size() != 2)
      return fail(RKV_ERR_INVALID_ARG, "safetensors: malformed entry for '" + e.name + "'");
    if (dt->str != "F32")  // rustral_io reads F32 only (crates/io/src/lib.rs:151-160)
      return fail(RKV_ERR_INVALID_ARG,
                  "dtype mismatch for '" + e.name + "': expected F32, got " + dt->str);
    std::vector<int64_t> shape;
    for (const Json& x : sh->arr) {
      if (x.kind != Json::Num || !(x.num >= 0 && x.num <= 1099511627776.0))  // 2^40
        return fail(RKV_ERR_INVALID_ARG, "safetensors: bad shape for '" + e.name + "'");
      shape.push_back((int64_t)x.num);
    }
    if (shape != e.shape)
      return fail(RKV_ERR_INVALID_ARG, "load_model: shape mismatch for '" + e.name +
                                           "': expected " + shape_str(e.shape) + ", got " +
                                           shape_str(shape));
    int64_t count = 1;
    for (int64_t s : shape) count *= s;
    if (off->arr[0].kind != Json::Num || off->arr[1].kind != Json::Num)
      return fail(RKV_ERR_INVALID_ARG, "safetensors: bad data_offsets for '" + e.name + "'");
    const double b0 = off->arr[0].num, b1 = off->arr[1].num;
    if (b0 < 0 || b1 < b0 || b1 > (double)body_len || (uint64_t)(b1 - b0) != (uint64_t)count * 4)
      return fail(RKV_ERR_INVALID_ARG, "safetensors: bad data_offsets for '" + e.name + "'");
    std::memcpy(host_params + e.offset, body + (uint64_t)b0, (size_t)count * 4);  // little endian
  }
  return RKV_OK;
}

extern "C" int rkv_decoder_save_safetensors(const rkv_decoder_config* cfg,
                                            const float* host_params, int64_t n_params,
                                            const char* path) {
  rkv::clear_error();
  if (!rkv::config_ok(cfg) || !path || !host_params)
    return fail(RKV_ERR_INVALID_ARG, "rkv_decoder_save_safetensors: bad argument");
  if (n_params != rkv::param_count(*cfg))
    return fail(RKV_ERR_INVALID_ARG,
                "rkv_decoder_save_safetensors: n_params does not match rkv_decoder_param_count");
  const std::vector<Entry> es = layout(*cfg);
  std::string h = "{";
  uint64_t pos = 0;
  for (size_t i = 0; i < es.size(); ++i) {
    int64_t count = 1;
    for (int64_t s : es[i].shape) count *= s;
    std::string shape = "[";
    for (size_t k = 0; k < es[i].shape.size(); ++k)
      shape += (k ? "," : "") + std::to_string(es[i].shape[k]);
    shape += "]";
    h += (i ? "," : "") + std::string("\"") + json_escape(es[i].name) + "\":{\"dtype\":\"F32\"," +
         "\"shape\":" + shape + ",\"data_offsets\":[" + std::to_string(pos) + "," +
         std::to_string(pos + (uint64_t)count * 4) + "]}";
    pos += (uint64_t)count * 4;
  }
  h += ",\"__metadata__\":{\"format\":\"rustral-decoder\"}}";
  while (h.size() % 8) h += ' ';  // keep the data 8-byte aligned
  FILE* f = std::fopen(path, "wb");
  if (!f) return fail(RKV_ERR_INVALID_ARG, std::string("cannot create ") + path);
  uint8_t len[8];
  for (int i = 0; i < 8; ++i) len[i] = (uint8_t)((uint64_t)h.size() >> (8 * i));
  bool ok = std::fwrite(len, 1, 8, f) == 8 && std::fwrite(h.data(), 1, h.size(), f) == h.size();
  for (size_t i = 0; ok && i < es.size(); ++i) {
    int64_t count = 1;
    for (int64_t s : es[i].shape) count *= s;
    ok = std::fwrite(host_params + es[i].offset, 4, (size_t)count, f) == (size_t)count;
  }
  ok = (std::fclose(f) == 0) && ok;
  if (!ok) return fail(RKV_ERR_INVALID_ARG, std::string("write error on ") + path);
  return RKV_OK;
}
