// Host-only fuzz driver for the safetensors reader (safetensors.cpp), built
// with AddressSanitizer and UndefinedBehaviorSanitizer by
// tests/test_safetensors_fuzz.py.  Test infrastructure, not product code.
//
// usage: safetensors_fuzz <seed file> <work file> <iterations>
// Each iteration writes a mutation of the seed file (truncation, random
// bytes anywhere, random bytes in the header, JSON punctuation in the
// header) and runs it through rkv_st_open / rkv_st_tensor and the decoder's
// strict load; every call must return normally (accepted or rejected).
#include <cstdio>
#include <cstdlib>
#include <random>
#include <string>
#include <vector>

#include "../../include/rustral_model.h"
#include "../../rustral_amd/csrc/model_layout.hpp"

namespace rkv {
void set_error(const std::string&) {}
void clear_error() {}
}  // namespace rkv

int main(int argc, char** argv) {
  if (argc != 4) return 2;
  const rkv_decoder_config c{50, 64, 4, 2, 96, 2, 32, 1e-5f};
  const int64_t n = rkv::param_count(c);
  std::vector<float> q((size_t)n);
  std::vector<unsigned char> good;
  FILE* f = std::fopen(argv[1], "rb");
  if (!f) return 2;
  for (int ch; (ch = std::fgetc(f)) != EOF;) good.push_back((unsigned char)ch);
  std::fclose(f);
  if (good.size() < 16) return 2;
  std::mt19937 rng(1);
  const int iters = std::atoi(argv[3]);
  int ok = 0, rejected = 0;
  static const char kPunct[] = "{}[]\":,0123456789-e.\\u";
  for (int it = 0; it < iters; ++it) {
    std::vector<unsigned char> m = good;
    const int kind = (int)(rng() % 4);
    if (kind == 0) {
      m.resize(rng() % m.size());
    } else {
      const size_t hdr = std::min<size_t>((size_t)(m[0] | (m[1] << 8)) + 8, m.size());
      const int nmut = 1 + (int)(rng() % 8);
      for (int k = 0; k < nmut; ++k) {
        const size_t pos = kind == 1 ? rng() % m.size() : rng() % hdr;
        m[pos] = (unsigned char)(kind == 3 ? kPunct[rng() % (sizeof kPunct - 1)] : rng());
      }
    }
    FILE* g = std::fopen(argv[2], "wb");
    if (!g) return 2;
    std::fwrite(m.data(), 1, m.size(), g);
    std::fclose(g);
    rkv_st_file* h = rkv_st_open(argv[2]);
    if (h) {
      for (int64_t i = 0; i < rkv_st_num_tensors(h); ++i) {
        const char *name = nullptr, *dt = nullptr;
        int nd = 0;
        int64_t shape[8];
        if (rkv_st_tensor(h, i, &name, &dt, &nd, shape, 8) == 0 && (!name || !dt)) return 3;
      }
      rkv_st_close(h);
    }
    (rkv_decoder_load_safetensors(&c, argv[2], q.data(), n) == 0 ? ok : rejected)++;
  }
  std::printf("accepted %d rejected %d\n", ok, rejected);
  return 0;
}
