// capi.hip -- error state and version of the C ABI (include/rustral_kv.h).
#include <string>

#include "common.hpp"

namespace rkv {
namespace {
thread_local std::string g_last_error;
}
void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }
}  // namespace rkv

extern "C" const char* rkv_last_error(void) { return rkv::g_last_error.c_str(); }

extern "C" int rkv_version(void) { return 100; /* 0.1.0 */ }
