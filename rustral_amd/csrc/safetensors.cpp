// safetensors.cpp -- the safetensors reader (safetensors.hpp), the strict
// load of the reference's load_model, and the decoder's host loader and
// writer (include/rustral_model.h).  Host code only.
#include "safetensors.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <set>
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

std::string json_escape(const std::string& s) {
  std::string r;
  for (char ch : s) {
    if (ch == '"' || ch == '\\') r += '\\';
    r += ch;
  }
  return r;
}

int64_t dtype_size(const std::string& dt) {
  if (dt == "F64" || dt == "I64" || dt == "U64") return 8;
  if (dt == "F32" || dt == "I32" || dt == "U32") return 4;
  if (dt == "F16" || dt == "BF16" || dt == "I16" || dt == "U16") return 2;
  if (dt == "I8" || dt == "U8" || dt == "BOOL" || dt == "F8_E4M3" || dt == "F8_E5M2") return 1;
  return 0;  // unknown: the byte count is not checked
}

}  // namespace

namespace rkv {
namespace st {

File::~File() {
  if (map) munmap(map, map_len);
}

const Tensor* File::find(const std::string& name) const {
  for (const Tensor& t : tensors)
    if (t.name == name) return &t;
  return nullptr;
}

std::string shape_str(const std::vector<int64_t>& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

std::unique_ptr<File> open(const char* path, std::string& err) {
  std::unique_ptr<File> f(new File);
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) {
    err = std::string("cannot open ") + path + ": " + std::strerror(errno);
    return nullptr;
  }
  struct stat sb;
  if (fstat(fd, &sb) != 0) {
    err = std::string("cannot stat ") + path + ": " + std::strerror(errno);
    ::close(fd);
    return nullptr;
  }
  const size_t size = (size_t)sb.st_size;
  if (size < 8) {
    ::close(fd);
    err = "safetensors: file shorter than 8 bytes";
    return nullptr;
  }
  void* m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) {
    err = std::string("cannot map ") + path + ": " + std::strerror(errno);
    return nullptr;
  }
  f->map = m;
  f->map_len = size;
  const uint8_t* bytes = static_cast<const uint8_t*>(m);
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | bytes[i];
  if (hlen > size - 8) {
    err = "safetensors: header past the end";
    return nullptr;
  }
  Parser ps{reinterpret_cast<const char*>(bytes) + 8, reinterpret_cast<const char*>(bytes) + 8 + hlen};
  Json root;
  if (!ps.value(root, 0) || root.kind != Json::Obj) {
    err = "safetensors: header is not a JSON object";
    return nullptr;
  }
  ps.ws();  // the writer pads the header with spaces; anything else after it is an error
  if (ps.p != ps.end) {
    err = "safetensors: trailing characters after the header object";
    return nullptr;
  }
  f->data = bytes + 8 + hlen;
  f->data_len = size - 8 - hlen;
  std::set<std::string> seen;
  for (const auto& kv : root.obj) {
    if (kv.first == "__metadata__") continue;
    const std::string& name = kv.first;
    if (!seen.insert(name).second) {
      err = "safetensors: duplicate entry '" + name + "'";
      return nullptr;
    }
    const Json *dt = nullptr, *sh = nullptr, *off = nullptr;
    if (kv.second.kind == Json::Obj)
      for (const auto& e : kv.second.obj) {
        if (e.first == "dtype") dt = &e.second;
        if (e.first == "shape") sh = &e.second;
        if (e.first == "data_offsets") off = &e.second;
      }
    if (!dt || !sh || !off || dt->kind != Json::Str || sh->kind != Json::Arr ||
        off->kind != Json::Arr || off->arr.size() != 2) {
      err = "safetensors: malformed entry for '" + name + "'";
      return nullptr;
    }
    Tensor t;
    t.name = name;
    t.dtype = dt->str;
    double count = 1;
    for (const Json& x : sh->arr) {
      if (x.kind != Json::Num || !(x.num >= 0 && x.num <= 1099511627776.0) ||  // 2^40
          x.num != (double)(int64_t)x.num) {
        err = "safetensors: bad shape for '" + name + "'";
        return nullptr;
      }
      t.shape.push_back((int64_t)x.num);
      count *= x.num;
    }
    const Json &o0 = off->arr[0], &o1 = off->arr[1];
    const int64_t es = dtype_size(t.dtype);
    if (o0.kind != Json::Num || o1.kind != Json::Num || !(o0.num >= 0) || o1.num < o0.num ||
        o1.num > (double)f->data_len || o0.num != (double)(uint64_t)o0.num ||
        o1.num != (double)(uint64_t)o1.num || count > 1e15 ||
        (es > 0 && (o1.num - o0.num) != count * (double)es)) {
      err = "safetensors: bad data_offsets for '" + name + "'";
      return nullptr;
    }
    t.begin = (uint64_t)o0.num;
    t.end = (uint64_t)o1.num;
    f->tensors.push_back(std::move(t));
  }
  // The byte buffer is exactly the tensors' ranges laid end to end (the
  // safetensors format's validation): sorted by offset, each begins where the
  // previous ends, the first at 0 and the last at the end of the data -- no
  // overlap, no gap, no trailing bytes.
  std::vector<const Tensor*> order;
  for (const Tensor& t : f->tensors) order.push_back(&t);
  std::stable_sort(order.begin(), order.end(), [](const Tensor* a, const Tensor* b) {
    return a->begin != b->begin ? a->begin < b->begin : a->end < b->end;
  });
  uint64_t at = 0;
  for (const Tensor* t : order) {
    if (t->begin != at) {
      err = "safetensors: data of '" + t->name + "' " +
            (t->begin < at ? "overlaps the previous tensor" : "leaves a gap after the previous tensor");
      return nullptr;
    }
    at = t->end;
  }
  if (at != f->data_len) {
    err = "safetensors: " + std::to_string(f->data_len - at) +
          " data bytes past the last tensor";
    return nullptr;
  }
  return f;
}

bool match(const File& f, const std::vector<Want>& want, std::vector<const Tensor*>& found,
           std::string& err) {
  std::map<std::string, const Tensor*> by_name;
  for (const Tensor& t : f.tensors) by_name[t.name] = &t;
  std::set<std::string> wanted;
  std::string missing, extra;
  for (const Want& w : want) {
    wanted.insert(w.name);
    if (!by_name.count(w.name)) missing += (missing.empty() ? "" : ", ") + w.name;
  }
  if (!missing.empty()) {
    err = "load_model: missing keys: " + missing;
    return false;
  }
  for (const auto& kv : by_name)
    if (!wanted.count(kv.first)) extra += (extra.empty() ? "" : ", ") + kv.first;
  if (!extra.empty()) {
    err = "load_model: unexpected extra keys: " + extra;
    return false;
  }
  found.clear();
  for (const Want& w : want) {
    const Tensor* t = by_name[w.name];
    if (t->dtype != "F32") {  // rustral_io reads F32 only (crates/io/src/lib.rs:151-160)
      err = "dtype mismatch for '" + w.name + "': expected F32, got " + t->dtype;
      return false;
    }
    if (t->shape != w.shape) {
      err = "load_model: shape mismatch for '" + w.name + "': expected " + shape_str(w.shape) +
            ", got " + shape_str(t->shape);
      return false;
    }
    found.push_back(t);
  }
  return true;
}

std::vector<Want> decoder_layout(const rkv_decoder_config& c, std::vector<int64_t>* offsets) {
  const int64_t d = c.d_model, V = c.vocab, f = c.d_ff;
  const int64_t kvd = (int64_t)c.n_kv_heads * (d / c.n_heads);
  std::vector<Want> e;
  std::vector<int64_t> o;
  auto add = [&](const std::string& n, std::vector<int64_t> shape, int64_t off) {
    e.push_back({n, std::move(shape)});
    o.push_back(off);
  };
  add("token_embedding.weight", {V, d}, 0);
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerOffsets lo = layer_offsets(c, l);
    const std::string p = "layers." + std::to_string(l) + ".";
    add(p + "norm1.weight", {d}, lo.ln1_g);
    add(p + "norm1.bias", {d}, lo.ln1_b);
    add(p + "self_attn.q_proj.weight", {d, d}, lo.wq);
    add(p + "self_attn.q_proj.bias", {d}, lo.bq);
    add(p + "self_attn.k_proj.weight", {kvd, d}, lo.wk);
    add(p + "self_attn.k_proj.bias", {kvd}, lo.bk);
    add(p + "self_attn.v_proj.weight", {kvd, d}, lo.wv);
    add(p + "self_attn.v_proj.bias", {kvd}, lo.bv);
    add(p + "self_attn.out_proj.weight", {d, d}, lo.wo);
    add(p + "self_attn.out_proj.bias", {d}, lo.bo);
    add(p + "norm2.weight", {d}, lo.ln2_g);
    add(p + "norm2.bias", {d}, lo.ln2_b);
    add(p + "ff_linear1.weight", {f, d}, lo.w1);
    add(p + "ff_linear1.bias", {f}, lo.b1);
    add(p + "ff_linear2.weight", {d, f}, lo.w2);
    add(p + "ff_linear2.bias", {d}, lo.b2);
  }
  const int64_t fin = layer_offsets(c, c.n_layers - 1).end;
  add("final_norm.weight", {d}, fin);
  add("final_norm.bias", {d}, fin + d);
  add("lm_head.weight", {V, d}, fin + 2 * d);
  if (offsets) *offsets = std::move(o);
  return e;
}

}  // namespace st
}  // namespace rkv

using rkv::st::File;

extern "C" rkv_st_file* rkv_st_open(const char* path) {
  rkv::clear_error();
  if (!path) {
    set_error("rkv_st_open: null path");
    return nullptr;
  }
  std::string err;
  std::unique_ptr<File> f = rkv::st::open(path, err);
  if (!f) {
    set_error(err);
    return nullptr;
  }
  rkv_st_file* h = new rkv_st_file;
  h->f = std::move(f);
  return h;
}

extern "C" void rkv_st_close(rkv_st_file* f) { delete f; }

extern "C" int64_t rkv_st_num_tensors(const rkv_st_file* f) {
  return f ? (int64_t)f->f->tensors.size() : -1;
}

extern "C" int rkv_st_tensor(const rkv_st_file* f, int64_t i, const char** name,
                             const char** dtype, int* ndim, int64_t* shape, int max_dims) {
  rkv::clear_error();
  if (!f || i < 0 || i >= (int64_t)f->f->tensors.size())
    return fail(RKV_ERR_INVALID_ARG, "rkv_st_tensor: no such tensor");
  const rkv::st::Tensor& t = f->f->tensors[(size_t)i];
  if (name) *name = t.name.c_str();
  if (dtype) *dtype = t.dtype.c_str();
  if (ndim) *ndim = (int)t.shape.size();
  if (shape) {
    if ((int)t.shape.size() > max_dims)
      return fail(RKV_ERR_INVALID_ARG, "rkv_st_tensor: more dimensions than max_dims");
    for (size_t k = 0; k < t.shape.size(); ++k) shape[k] = t.shape[k];
  }
  return RKV_OK;
}

extern "C" int rkv_decoder_load_safetensors(const rkv_decoder_config* cfg, const char* path,
                                            float* host_params, int64_t n_params) {
  rkv::clear_error();
  if (!rkv::config_ok(cfg) || !path || !host_params)
    return fail(RKV_ERR_INVALID_ARG, "rkv_decoder_load_safetensors: bad argument");
  if (n_params != rkv::param_count(*cfg))
    return fail(RKV_ERR_INVALID_ARG,
                "rkv_decoder_load_safetensors: n_params does not match rkv_decoder_param_count");
  std::string err;
  std::unique_ptr<File> f = rkv::st::open(path, err);
  if (!f) return fail(RKV_ERR_INVALID_ARG, err);
  std::vector<int64_t> offsets;
  const std::vector<rkv::st::Want> want = rkv::st::decoder_layout(*cfg, &offsets);
  std::vector<const rkv::st::Tensor*> found;
  if (!rkv::st::match(*f, want, found, err)) return fail(RKV_ERR_INVALID_ARG, err);
  for (size_t i = 0; i < want.size(); ++i)  // little-endian F32, as stored
    std::memcpy(host_params + offsets[i], f->data + found[i]->begin,
                (size_t)(found[i]->end - found[i]->begin));
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
  std::vector<int64_t> offsets;
  const std::vector<rkv::st::Want> es = rkv::st::decoder_layout(*cfg, &offsets);
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
    ok = std::fwrite(host_params + offsets[i], 4, (size_t)count, f) == (size_t)count;
  }
  ok = (std::fclose(f) == 0) && ok;
  if (!ok) return fail(RKV_ERR_INVALID_ARG, std::string("write error on ") + path);
  return RKV_OK;
}
