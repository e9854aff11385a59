// common.hpp -- shared device helpers and host error plumbing for
// librustral_kv.so (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/rustral_kv.h"

namespace rkv {

// ---- host-side error reporting -------------------------------------------

void set_error(const std::string& msg);
void clear_error();

inline int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

// Checks the launch just enqueued; maps a HIP failure to RKV_ERR_HIP.
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(RKV_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return RKV_OK;
}

inline size_t elem_size(int dtype) { return dtype == RKV_F32 ? 4 : 2; }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- bf16 ----------------------------------------------------------------

// fp32 -> bf16, round to nearest even; NaN keeps sign/payload with the quiet
// bit set.  The oracle uses the same bit routine (oracle/rkv_oracle.c).
__device__ __forceinline__ uint32_t bf16_rne(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Packs two floats into one dword of bf16 (lo = a, hi = b).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return bf16_rne(a) | (bf16_rne(b) << 16);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ---- cross-lane sums (wave64) --------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Sum over aligned groups of N consecutive lanes; every lane of the group
// receives the group total.  N in {1,2,4,8,16,32,64}.
// Steps 1..8 use DPP inside a 16-lane row: quad_perm xor1 (0xB1), quad_perm
// xor2 (0x4E), row_half_mirror (0x141), row_mirror (0x140).  After the quad
// steps all four lanes of a quad hold the same value, so a mirror pairs each
// lane with a lane of the other half and the sum is complete.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += dpp<0xB1>(x);
  if constexpr (N >= 4) x += dpp<0x4E>(x);
  if constexpr (N >= 8) x += dpp<0x141>(x);
  if constexpr (N >= 16) x += dpp<0x140>(x);
  if constexpr (N >= 32) x += __shfl_xor(x, 16);
  if constexpr (N >= 64) x += __shfl_xor(x, 32);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

}  // namespace rkv
