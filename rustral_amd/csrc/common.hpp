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
// Written with a select, not an early return: a data-dependent branch per
// element costs an exec-mask region in every caller.
__device__ __forceinline__ uint32_t bf16_rne(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t nan = (u >> 16) | 0x40u;
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return (u & 0x7fffffffu) > 0x7f800000u ? nan : rounded;
}

// Packs two floats into one dword of bf16 (lo = a, hi = b).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return bf16_rne(a) | (bf16_rne(b) << 16);
}

// ---- streaming memory access ----------------------------------------------
// 16-byte load / store with the nontemporal hint (the `nt` bit): KV bytes
// are touched once per call, and marking them as streaming keeps them from
// displacing reusable lines in L2 and the Infinity Cache.  On gfx950 a
// decode-shaped stream of 4 KiB tiles reads ~12% faster this way
// (5.6 -> 6.35 TB/s measured for the configs[2] access pattern).
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 load_stream(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(static_cast<const u32x4_t*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void store_stream(void* p, const uint4& w) {
  const u32x4_t v = {w.x, w.y, w.z, w.w};
  __builtin_nontemporal_store(v, static_cast<u32x4_t*>(p));
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ---- 1-byte KV storage: int8 and OCP fp8 e4m3 with a per-row scale ---------
// A row (the D elements of one token of one KV head) is stored as D bytes
// plus one fp32 scale s:
//   int8: amax = max |x|; s = amax / 127; q = rint(x * (127 / amax)) clamped
//         to [-127, 127] (amax = 0 or x NaN: q = 0); value = q * s.
//   fp8:  s = amax / 448; q = e4m3(x * (448 / amax)), round to nearest even,
//         magnitudes >= 448 saturate to 448, NaN stays NaN; value = f(q) * s.
// The oracle uses the same bit routines (oracle/rkv_oracle.c), so the stored
// bytes and scales match exactly.

__host__ __device__ __forceinline__ uint8_t i8_quant(float x, float inv) {
  const float r = rintf(x * inv);
  if (!(r == r)) return 0;  // NaN
  const float c = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
  return (uint8_t)(int8_t)(int)c;
}

__host__ __device__ __forceinline__ uint8_t e4m3_from_f32(float x) {
  uint32_t u;
  __builtin_memcpy(&u, &x, 4);
  const uint32_t sign = (u >> 24) & 0x80u, a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7fu);     // NaN
  if (a >= 0x43e00000u) return (uint8_t)(sign | 0x7eu);    // >= 448: saturate
  if (a < 0x3c800000u) {                                   // below 2^-6: subnormal
    float f;
    __builtin_memcpy(&f, &a, 4);
    return (uint8_t)(sign | (uint32_t)(int)rintf(f * 512.0f));  // m * 2^-9, m <= 8
  }
  uint32_t e = (a >> 23) - 120u;  // biased e4m3 exponent, 1..15
  uint32_t m = (a >> 20) & 7u;
  const uint32_t rem = a & 0xfffffu;
  if (rem > 0x80000u || (rem == 0x80000u && (m & 1u))) ++m;  // round to nearest even
  if (m == 8u) {
    m = 0;
    ++e;
  }
  return (uint8_t)(sign | (e << 3) | m);
}

// Exact: the 7 exponent + mantissa bits placed at f32 bit 20 form a float
// 2^(e-127) (1 + m/8) -- or the subnormal m 2^-129 when e = 0 -- and the
// power-of-two factor 2^120 moves the bias from 127 to e4m3's 7.  (Relies on
// fp32 denormals being kept, the default float mode of these kernels.)
__host__ __device__ __forceinline__ float f32_from_e4m3(uint8_t b) {
  const uint32_t mag = b & 0x7fu;
  uint32_t u = mag << 20;
  float f;
  __builtin_memcpy(&f, &u, 4);
  f *= 1.329227995784916e36f;  // 2^120
  __builtin_memcpy(&u, &f, 4);
  if (mag == 0x7fu) u = 0x7fc00000u;  // NaN
  u |= (uint32_t)(b & 0x80u) << 24;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

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
  if constexpr (N >= 32) {
    const auto r =
        __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if constexpr (N >= 64) {
    const auto r =
        __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  return x;
}

// Maximum over aligned groups of N consecutive lanes (N in {4, 8, 16}); every
// lane of the group receives it.
template <int N>
__device__ __forceinline__ float group_max(float x) {
  if constexpr (N >= 2) x = fmaxf(x, dpp<0xB1>(x));
  if constexpr (N >= 4) x = fmaxf(x, dpp<0x4E>(x));
  if constexpr (N >= 8) x = fmaxf(x, dpp<0x141>(x));
  if constexpr (N >= 16) x = fmaxf(x, dpp<0x140>(x));
  return x;
}

// Two floats to packed bf16 (a in the low half), round to nearest even: one
// v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint32_t cvt_bf16x2(float a, float b) {
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
  typedef __attribute__((ext_vector_type(2))) float f32x2_t;
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{a, b}), bf16x2_t));
}

// Transposing LDS reads of gfx950 (lane mappings probed on the GPU).
// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives as
// element j (j < 4) the 16-bit element i & 3 of the 8 bytes addressed by lane
// 4 j + (i >> 2).  So when lane i of group g addresses row 4 g + (i >> 2),
// columns c0 + 4 (i & 3) .. + 3 of a row-major 16-bit tile, it receives
// column c0 + i of rows 4 g .. 4 g + 3.
__device__ __forceinline__ uint2 lds_read_tr16(const void* p) {
  typedef __attribute__((ext_vector_type(4))) short i16x4_t;
  typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
  return __builtin_bit_cast(
      uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)const_cast<void*>(p)));
}
// ds_read_b64_tr_b8: within each group of 16 lanes, lane i receives as byte j
// (j < 8) byte i & 7 of the 8 bytes addressed by lane 2 j + (i >> 3).  So when
// lane i of group g addresses row 8 g + (i >> 1), bytes c0 + 8 (i & 1) .. + 7
// of a row-major byte tile, it receives column c0 + i of rows 8 g .. 8 g + 7.
__device__ __forceinline__ uint2 lds_read_tr8(const void* p) {
  typedef __attribute__((ext_vector_type(2))) int i32x2_t;
  typedef __attribute__((address_space(3))) i32x2_t lds_i32x2;
  return __builtin_bit_cast(
      uint2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)const_cast<void*>(p)));
}

// x[l] + x[l ^ 16] and x[l] + x[l ^ 32] through v_permlane16_swap /
// v_permlane32_swap (VALU, no LDS round trip).  Called with the same value
// twice, a swap returns the pair (x[l], x[l ^ 16]) in some order, so the sum
// (commutative) is the bits of x + __shfl_xor(x, 16).
__device__ __forceinline__ float pair16_sum(float x) {
  const auto r =
      __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair32_sum(float x) {
  const auto r =
      __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair16_max(float x) {
  const auto r =
      __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair32_max(float x) {
  const auto r =
      __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Maximum / sum over the 64 lanes, every lane receiving it: DPP inside each
// 16-lane row, then the row pairs by permlane swaps.
__device__ __forceinline__ float wave_max(float x) {
  return pair32_max(pair16_max(group_max<16>(x)));
}

__device__ __forceinline__ float wave_sum(float x) {
  return pair32_sum(pair16_sum(group_sum<16>(x)));
}

}  // namespace rkv
