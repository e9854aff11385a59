// ceiling.hip -- what HBM streams at on this part, for the access patterns of
// the paged-KV kernels: a measurement library (librkv_ceiling.so), not part
// of the product ABI.  The kernels move bytes and do no arithmetic beyond
// folding what they read into a value that is stored only when it equals a
// runtime argument (so the loads cannot be dropped).
//
//   rkvc_read         flat read, nontemporal 16-byte loads, grid-stride
//   rkvc_write        flat write, 16-byte stores, grid-stride
//   rkvc_copy         flat copy, nontemporal loads and stores
//   rkvc_write_var    flat write variants: store policy, vectors per lane,
//   rkvc_copy_var     interleaved or contiguous per workgroup (and load
//                     policy for copies), at any grid size
//   rkvc_block_copy   one workgroup per (src, dst) pair of fixed-size blocks
//                     within one pool (the copy_blocks pattern)
//   rkvc_tile_stream  the decode kernel's loads alone: grid (Hkv, partitions,
//                     sequences), 4 waves per 640-token partition, each wave
//                     streaming 10 K then 10 V (block, head) tiles of
//                     D = 128 (bf16, or 1-byte with row scales) through a
//                     ring of 4 tiles, 1 KiB of whole rows per wave-load,
//                     tiles past the context re-reading the wave's first
//                     tile
//   rkvc_tile_stream_shape  the bf16 decode pattern at the 768- and 1280-token
//                     8-wave partition shapes
//   rkvc_nth          write, copy and block copy, one 16-byte unit a thread,
//                     by workgroup size (64 to 512 threads)
//   rkvc_tile_stream_1b  variants of the 1-byte pattern: no scales, 2 or 4
//                     KV heads per wave, a partition-major grid, the scales
//                     in a 128-byte line after each K tile
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ u32x4 ld(const u32x4* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <bool NT>
__device__ __forceinline__ void st(u32x4* p, u32x4 v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}
__device__ __forceinline__ unsigned fold(u32x4 a) { return a[0] ^ a[1] ^ a[2] ^ a[3]; }

template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

constexpr int kUnr = 8;

__global__ __launch_bounds__(256) void read_kernel(const u32x4* __restrict__ s, int64_t n,
                                                   unsigned* sink, unsigned magic) {
  const int64_t stride = (int64_t)gridDim.x * 256 * kUnr;
  unsigned acc = 0;
  for (int64_t u0 = (int64_t)blockIdx.x * 256 * kUnr + threadIdx.x; u0 < n; u0 += stride) {
#pragma unroll
    for (int k = 0; k < kUnr; ++k) {
      const int64_t u = u0 + k * 256;
      if (u < n) acc ^= fold(ld<true>(s + u));
    }
  }
  if (acc == magic) sink[0] = acc;
}

__global__ __launch_bounds__(256) void write_kernel(u32x4* __restrict__ d, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256 * kUnr;
  const u32x4 v = {threadIdx.x, blockIdx.x, 0x3f800000u, 0u};
  for (int64_t u0 = (int64_t)blockIdx.x * 256 * kUnr + threadIdx.x; u0 < n; u0 += stride) {
#pragma unroll
    for (int k = 0; k < kUnr; ++k) {
      const int64_t u = u0 + k * 256;
      if (u < n) st<false>(d + u, v);
    }
  }
}

__global__ __launch_bounds__(256) void copy_kernel(const u32x4* __restrict__ s,
                                                   u32x4* __restrict__ d, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256 * kUnr;
  for (int64_t u0 = (int64_t)blockIdx.x * 256 * kUnr + threadIdx.x; u0 < n; u0 += stride) {
    u32x4 x[kUnr];
#pragma unroll
    for (int k = 0; k < kUnr; ++k) {
      const int64_t u = u0 + k * 256;
      if (u < n) x[k] = ld<true>(s + u);
    }
#pragma unroll
    for (int k = 0; k < kUnr; ++k) {
      const int64_t u = u0 + k * 256;
      if (u < n) st<true>(d + u, x[k]);
    }
  }
}

__global__ __launch_bounds__(256) void block_copy_kernel(char* __restrict__ pool,
                                                         const int32_t* __restrict__ pairs,
                                                         int64_t block_bytes, int64_t num_blocks) {
  const int32_t src = pairs[2 * blockIdx.x], dst = pairs[2 * blockIdx.x + 1];
  if (src < 0 || src >= num_blocks || dst < 0 || dst >= num_blocks) return;
  const u32x4* s = reinterpret_cast<const u32x4*>(pool + src * block_bytes);
  u32x4* d = reinterpret_cast<u32x4*>(pool + dst * block_bytes);
  const int64_t n = block_bytes >> 4;
  for (int64_t u0 = threadIdx.x; u0 < n; u0 += kUnr * 256) {
    u32x4 x[kUnr];
#pragma unroll
    for (int k = 0; k < kUnr; ++k) {
      const int64_t u = u0 + k * 256;
      if (u < n) x[k] = ld<true>(s + u);
    }
#pragma unroll
    for (int k = 0; k < kUnr; ++k) {
      const int64_t u = u0 + k * 256;
      if (u < n) st<true>(d + u, x[k]);
    }
  }
}

// D = 128, 16-token blocks.  EB = 2 (bf16): a (block, head) tile is 4 KiB,
// four 256-byte rows per wave-load.  EB = 1 (1-byte pools): a tile is 2 KiB,
// eight 128-byte rows per wave-load, plus the fp32 row scales the decode
// kernel reads (one K scale per lane and K tile, the V scales of the wave's
// slice up front).
// NTW tiles a wave and SPLIT waves a workgroup (partitions of 16 NTW SPLIT
// tokens): 10 x 4 (640) is the decode kernel's 4-wave build, 6 x 8 (768) and
// 10 x 8 (1280) its 8-wave builds.
constexpr int kD = 128, kBS = 16, kNTW = 10, kR = 4, kSplit = 4;
constexpr int kP = kNTW * kSplit * kBS;  // tokens per partition of the 1-byte variants (640)

template <int EB, int NTW = kNTW, int SPLIT = kSplit>
__global__ __launch_bounds__(64 * SPLIT) void tile_stream_kernel(
    const uint8_t* __restrict__ k_pool, const uint8_t* __restrict__ v_pool,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale,
    const int32_t* __restrict__ tables, int max_blocks, const int32_t* __restrict__ ctx_lens,
    int num_kv_heads, int64_t num_blocks, unsigned* sink, unsigned magic) {
  constexpr int ROW = kD * EB;          // bytes per token row
  constexpr int RPL = 1024 / ROW;       // rows per 1 KiB wave-load
  constexpr int NL = kBS / RPL;         // wave-loads per tile
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int kh = blockIdx.x, part = blockIdx.y, b = blockIdx.z;
  constexpr int P = NTW * SPLIT * kBS;
  const int L = ctx_lens[b];
  if (part * P >= L) return;
  const int lb0 = part * (P / kBS) + w * NTW;
  const int32_t* tab = tables + (int64_t)b * max_blocks;
  int32_t pb[NTW];
#pragma unroll
  for (int i = 0; i < NTW; ++i) {
    const int lb = lb0 + i;
    pb[i] = tab[lb < max_blocks ? lb : max_blocks - 1];
  }
  const int32_t pb0 = pb[0] >= 0 && pb[0] < num_blocks ? pb[0] : 0;
  int64_t row0[NTW];  // first token row of each (block, head) tile
#pragma unroll
  for (int i = 0; i < NTW; ++i) {
    const bool ok = (lb0 + i) * kBS < L && pb[i] >= 0 && pb[i] < num_blocks;
    row0[i] = ((int64_t)(ok ? pb[i] : pb0) * num_kv_heads + kh) * kBS;
  }
  const uint32_t off = (lane / (64 / RPL)) * ROW + (lane % (64 / RPL)) * 16;
  auto tile_load = [&](int t, int n) __attribute__((always_inline)) {
    const uint8_t* p = (t < NTW ? k_pool : v_pool) + row0[t % NTW] * ROW;
    return ld<true>(reinterpret_cast<const u32x4*>(p + off + n * 1024));
  };
  unsigned acc = 0;
  u32x4 ring[kR][NL];
#pragma unroll
  for (int t = 0; t < kR; ++t)
#pragma unroll
    for (int n = 0; n < NL; ++n) ring[t][n] = tile_load(t, n);
  float sc = 0.0f;
  if constexpr (EB == 1) {
#pragma unroll
    for (int i = 0; i < NTW; ++i) sc += k_scale[row0[i] + (lane & 15)];
#pragma unroll
    for (int j = 0; j < (NTW * kBS + 63) / 64; ++j) {
      const int x = lane + 64 * j;
      if (x < NTW * kBS) sc += v_scale[row0[x / kBS] + x % kBS];
    }
  }
  static_for<0, 2 * NTW>([&](auto tc) __attribute__((always_inline)) {
    constexpr int t = decltype(tc)::value;
#pragma unroll
    for (int n = 0; n < NL; ++n) acc ^= fold(ring[t % kR][n]) + t;
    if constexpr (t + kR < 2 * NTW) {
#pragma unroll
      for (int n = 0; n < NL; ++n) ring[t % kR][n] = tile_load(t + kR, n);
    }
    __builtin_amdgcn_sched_barrier(0);
  });
  acc += __float_as_uint(sc);
  if (acc == magic) sink[0] = acc;
}

// Variants of the 1-byte tile stream (same grid, 4 waves, 10 + 10 tiles a
// wave, ring of 4 wave-load pairs):
//   HPW  KV heads per wave: a (block, HPW heads) tile is HPW x 2 KiB of
//        contiguous rows, the grid has Hkv / HPW workgroups per (partition,
//        sequence) and the ring holds 4 / HPW tiles;
//   SC   0: no scales; 1: the row scales as the decode kernel reads them
//        (k_scale / v_scale [num_blocks][Hkv][16] fp32); 2: the K and V row
//        scales of a (block, head) in a 128-byte line right after its K tile
//        (the K pool then holds 2,176-byte tiles);
//   PM   partition-major grid (Hkv / HPW, sequences, partitions): every
//        sequence's first partition is dispatched before any second one.
template <int HPW, int SC, bool PM>
__global__ __launch_bounds__(64 * kSplit) void tile_stream1_kernel(
    const uint8_t* __restrict__ k_pool, const uint8_t* __restrict__ v_pool,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale,
    const int32_t* __restrict__ tables, int max_blocks, const int32_t* __restrict__ ctx_lens,
    int num_kv_heads, int64_t num_blocks, unsigned* sink, unsigned magic) {
  constexpr int NL = 2 * HPW, R = kR / HPW;
  constexpr int KT = SC == 2 ? kBS * kD + 128 : kBS * kD, VT = kBS * kD;  // tile strides
  static_assert(R >= 1, "ring of at least one tile");
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int kh = blockIdx.x * HPW;
  const int part = PM ? blockIdx.z : blockIdx.y, b = PM ? blockIdx.y : blockIdx.z;
  const int L = ctx_lens[b];
  if (part * kP >= L) return;
  const int lb0 = part * (kP / kBS) + w * kNTW;
  const int32_t* tab = tables + (int64_t)b * max_blocks;
  int32_t pb[kNTW];
#pragma unroll
  for (int i = 0; i < kNTW; ++i) {
    const int lb = lb0 + i;
    pb[i] = tab[lb < max_blocks ? lb : max_blocks - 1];
  }
  const int32_t pb0 = pb[0] >= 0 && pb[0] < num_blocks ? pb[0] : 0;
  int64_t tix[kNTW];  // (block, first head) tile index
#pragma unroll
  for (int i = 0; i < kNTW; ++i) {
    const bool ok = (lb0 + i) * kBS < L && pb[i] >= 0 && pb[i] < num_blocks;
    tix[i] = (int64_t)(ok ? pb[i] : pb0) * num_kv_heads + kh;
  }
  const uint32_t off = lane * 16;
  auto tile_load = [&](int t, int n) __attribute__((always_inline)) {
    // HPW > 1 only with SC != 2: the HPW tiles of a block are contiguous
    const uint8_t* p = t < kNTW ? k_pool + tix[t] * KT : v_pool + tix[t - kNTW] * VT;
    return ld<true>(reinterpret_cast<const u32x4*>(p + off + n * 1024));
  };
  unsigned acc = 0;
  u32x4 ring[R][NL];
#pragma unroll
  for (int t = 0; t < R; ++t)
#pragma unroll
    for (int n = 0; n < NL; ++n) ring[t][n] = tile_load(t, n);
  float sc = 0.0f;
  if constexpr (SC == 1) {
#pragma unroll
    for (int i = 0; i < kNTW; ++i) sc += k_scale[tix[i] * kBS + (lane & (16 * HPW - 1))];
#pragma unroll
    for (int j = 0; j < (kNTW * kBS * HPW + 63) / 64; ++j) {
      const int x = lane + 64 * j;
      if (x < kNTW * kBS * HPW) sc += v_scale[tix[x / (kBS * HPW)] * kBS + x % (kBS * HPW)];
    }
  } else if constexpr (SC == 2) {
#pragma unroll
    for (int i = 0; i < kNTW; ++i)
      sc += reinterpret_cast<const float*>(k_pool + tix[i] * KT + kBS * kD)[lane & 31];
  }
  static_for<0, 2 * kNTW>([&](auto tc) __attribute__((always_inline)) {
    constexpr int t = decltype(tc)::value;
#pragma unroll
    for (int n = 0; n < NL; ++n) acc ^= fold(ring[t % R][n]) + t;
    if constexpr (t + R < 2 * kNTW) {
#pragma unroll
      for (int n = 0; n < NL; ++n) ring[t % R][n] = tile_load(t + R, n);
    }
    __builtin_amdgcn_sched_barrier(0);
  });
  acc += __float_as_uint(sc);
  if (acc == magic) sink[0] = acc;
}

// Block copies with the next pair's loads in flight while the current
// pair's stores drain: workgroup g copies pairs g, g + grid, g + 2 grid, ...
// (32 KiB blocks: 256 threads x 8 x 16 bytes, one round per block).
__global__ __launch_bounds__(256) void block_copy_pipe_kernel(char* __restrict__ pool,
                                                              const int32_t* __restrict__ pairs,
                                                              int n_pairs, int64_t num_blocks) {
  constexpr int64_t kBlk = 32768;
  auto load = [&](int i, u32x4 (&x)[kUnr]) __attribute__((always_inline)) {
    int32_t src = pairs[2 * i];
    src = src >= 0 && src < num_blocks ? src : 0;
    const u32x4* s = reinterpret_cast<const u32x4*>(pool + src * kBlk);
#pragma unroll
    for (int k = 0; k < kUnr; ++k) x[k] = ld<true>(s + k * 256 + threadIdx.x);
  };
  int i = blockIdx.x;
  if (i >= n_pairs) return;
  u32x4 cur[kUnr], nxt[kUnr];
  load(i, cur);
  for (; i < n_pairs; i += gridDim.x) {
    const int j = i + gridDim.x;
    if (j < n_pairs) load(j, nxt);
    const int32_t src = pairs[2 * i], dst = pairs[2 * i + 1];
    if (src >= 0 && src < num_blocks && dst >= 0 && dst < num_blocks) {
      u32x4* d = reinterpret_cast<u32x4*>(pool + dst * kBlk);
#pragma unroll
      for (int k = 0; k < kUnr; ++k) st<true>(d + k * 256 + threadIdx.x, cur[k]);
    }
#pragma unroll
    for (int k = 0; k < kUnr; ++k) cur[k] = nxt[k];
  }
}

// Work per workgroup: UNR 16-byte units a thread (UNR * 4 KiB a workgroup),
// wave-contiguous 1 KiB stores; grid-stride, so a grid of n / (256 UNR)
// workgroups is one round each.
template <int UNR>
__global__ __launch_bounds__(256) void write_unr_kernel(u32x4* __restrict__ d, int64_t n) {
  const u32x4 v = {threadIdx.x, blockIdx.x, 0x3f800000u, 0u};
  const int64_t stride = (int64_t)gridDim.x * 256 * UNR;
  for (int64_t u0 = (int64_t)blockIdx.x * 256 * UNR + threadIdx.x; u0 < n; u0 += stride) {
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      const int64_t u = u0 + k * 256;
      if (u < n) st<false>(d + u, v);
    }
  }
}

template <int UNR>
__global__ __launch_bounds__(256) void read_unr_kernel(const u32x4* __restrict__ s, int64_t n,
                                                       unsigned* sink, unsigned magic) {
  const int64_t stride = (int64_t)gridDim.x * 256 * UNR;
  unsigned acc = 0;
  for (int64_t u0 = (int64_t)blockIdx.x * 256 * UNR + threadIdx.x; u0 < n; u0 += stride) {
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      const int64_t u = u0 + k * 256;
      if (u < n) acc ^= fold(ld<true>(s + u));
    }
  }
  if (acc == magic) sink[0] = acc;
}

template <int UNR, bool NT>
__global__ __launch_bounds__(256) void copy_unr_kernel(const u32x4* __restrict__ s,
                                                       u32x4* __restrict__ d, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256 * UNR;
  for (int64_t u0 = (int64_t)blockIdx.x * 256 * UNR + threadIdx.x; u0 < n; u0 += stride) {
    u32x4 x[UNR];
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      const int64_t u = u0 + k * 256;
      if (u < n) x[k] = ld<true>(s + u);
    }
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      const int64_t u = u0 + k * 256;
      if (u < n) st<NT>(d + u, x[k]);
    }
  }
}

// Block copies with B-byte pieces per workgroup: grid (pieces of a block,
// pairs), each workgroup one round of UNR units a thread.
template <int UNR>
__global__ __launch_bounds__(256) void block_copy_unr_kernel(char* __restrict__ pool,
                                                             const int32_t* __restrict__ pairs,
                                                             int64_t block_bytes,
                                                             int64_t num_blocks) {
  const int32_t src = pairs[2 * blockIdx.y], dst = pairs[2 * blockIdx.y + 1];
  if (src < 0 || src >= num_blocks || dst < 0 || dst >= num_blocks) return;
  const int64_t off = (int64_t)blockIdx.x * 256 * UNR;
  const u32x4* sp = reinterpret_cast<const u32x4*>(pool + src * block_bytes) + off;
  u32x4* dp = reinterpret_cast<u32x4*>(pool + dst * block_bytes) + off;
  u32x4 x[UNR];
#pragma unroll
  for (int k = 0; k < UNR; ++k) x[k] = ld<true>(sp + k * 256 + threadIdx.x);
#pragma unroll
  for (int k = 0; k < UNR; ++k) st<true>(dp + k * 256 + threadIdx.x, x[k]);
}

// One 16-byte unit a thread and NTH threads a workgroup, one round (the
// grid covers the buffer, or every piece of every pair, once): flat write,
// flat copy (nontemporal loads and stores) and block copies in pieces of
// 16 NTH bytes -- the work per workgroup by workgroup size.
template <int NTH>
__global__ __launch_bounds__(NTH) void write_nth_kernel(u32x4* __restrict__ d, int64_t n) {
  const int64_t u = (int64_t)blockIdx.x * NTH + threadIdx.x;
  if (u < n) st<false>(d + u, u32x4{threadIdx.x, blockIdx.x, 0x3f800000u, 0u});
}
template <int NTH>
__global__ __launch_bounds__(NTH) void copy_nth_kernel(const u32x4* __restrict__ s,
                                                       u32x4* __restrict__ d, int64_t n) {
  const int64_t u = (int64_t)blockIdx.x * NTH + threadIdx.x;
  if (u < n) st<true>(d + u, ld<true>(s + u));
}
template <int NTH>
__global__ __launch_bounds__(NTH) void block_copy_nth_kernel(char* __restrict__ pool,
                                                             const int32_t* __restrict__ pairs,
                                                             int64_t block_bytes,
                                                             int64_t num_blocks) {
  const int32_t src = pairs[2 * blockIdx.y], dst = pairs[2 * blockIdx.y + 1];
  if (src < 0 || src >= num_blocks || dst < 0 || dst >= num_blocks) return;
  const int64_t u = (int64_t)blockIdx.x * NTH + threadIdx.x;
  const u32x4 x = ld<true>(reinterpret_cast<const u32x4*>(pool + src * block_bytes) + u);
  st<true>(reinterpret_cast<u32x4*>(pool + dst * block_bytes) + u, x);
}

// Store and copy variants (the write side of every copy):
//   NT      nontemporal (streaming) stores instead of the default policy
//   VPL     16-byte vectors per lane per step: 1, or 2 adjacent (32 bytes)
//   CHUNK   each workgroup owns one contiguous 1/grid of the buffer instead
//           of the grid-stride interleave (a persistent grid of one or a few
//           workgroups per CU then walks long sequential runs)
// NTL (copies) selects nontemporal loads.  Every variant writes every
// 16-byte unit of the buffer exactly once.
template <bool NT, int VPL, bool CHUNK>
__global__ __launch_bounds__(256) void write_var_kernel(u32x4* __restrict__ d, int64_t n) {
  const u32x4 v = {threadIdx.x, blockIdx.x, 0x3f800000u, 0u};
  constexpr int64_t STEP = 256 * kUnr * VPL;  // units per workgroup round
  int64_t lo, hi, stride;
  if constexpr (CHUNK) {
    const int64_t per = (n + gridDim.x - 1) / gridDim.x;
    lo = (int64_t)blockIdx.x * per;
    hi = lo + per < n ? lo + per : n;
    stride = STEP;
  } else {
    lo = (int64_t)blockIdx.x * STEP;
    hi = n;
    stride = (int64_t)gridDim.x * STEP;
  }
  for (int64_t r = lo; r < hi; r += stride) {
#pragma unroll
    for (int k = 0; k < kUnr; ++k) {
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        const int64_t u = r + ((int64_t)k * 256 + threadIdx.x) * VPL + j;
        if (u < hi) st<NT>(d + u, v);
      }
    }
  }
}

template <bool NTL, bool NTS, int VPL, bool CHUNK>
__global__ __launch_bounds__(256) void copy_var_kernel(const u32x4* __restrict__ s,
                                                       u32x4* __restrict__ d, int64_t n) {
  constexpr int64_t STEP = 256 * kUnr * VPL;
  int64_t lo, hi, stride;
  if constexpr (CHUNK) {
    const int64_t per = (n + gridDim.x - 1) / gridDim.x;
    lo = (int64_t)blockIdx.x * per;
    hi = lo + per < n ? lo + per : n;
    stride = STEP;
  } else {
    lo = (int64_t)blockIdx.x * STEP;
    hi = n;
    stride = (int64_t)gridDim.x * STEP;
  }
  for (int64_t r = lo; r < hi; r += stride) {
    u32x4 x[kUnr][VPL];
#pragma unroll
    for (int k = 0; k < kUnr; ++k)
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        const int64_t u = r + ((int64_t)k * 256 + threadIdx.x) * VPL + j;
        if (u < hi) x[k][j] = ld<NTL>(s + u);
      }
#pragma unroll
    for (int k = 0; k < kUnr; ++k)
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        const int64_t u = r + ((int64_t)k * 256 + threadIdx.x) * VPL + j;
        if (u < hi) st<NTS>(d + u, x[k][j]);
      }
  }
}

// The launch's own status: an error left by an earlier runtime call of the
// process is cleared before the launch (clear_errors), so it is not
// reported as this launch's.  Returns 0 or the positive hipError_t code.
void clear_errors() { (void)hipGetLastError(); }
int launched() { return (int)hipGetLastError(); }

}  // namespace

extern "C" {

int rkvc_read(const void* src, int64_t bytes, unsigned* sink, unsigned magic, int grid,
              void* stream) {
  if (!src || !sink || bytes < 16 || (bytes & 15) || grid <= 0) return -1;
  clear_errors();
  read_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const u32x4*>(src), bytes >> 4, sink, magic);
  return launched();
}

int rkvc_write(void* dst, int64_t bytes, int grid, void* stream) {
  if (!dst || bytes < 16 || (bytes & 15) || grid <= 0) return -1;
  clear_errors();
  write_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(static_cast<u32x4*>(dst),
                                                                   bytes >> 4);
  return launched();
}

int rkvc_copy(const void* src, void* dst, int64_t bytes, int grid, void* stream) {
  if (!src || !dst || bytes < 16 || (bytes & 15) || grid <= 0) return -1;
  clear_errors();
  copy_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), bytes >> 4);
  return launched();
}

// variant bits: 1 NT stores, 2 two vectors per lane, 4 contiguous chunk per
// workgroup; copies add 8 for nontemporal loads.
int rkvc_write_var(void* dst, int64_t bytes, int grid, int variant, void* stream) {
  if (!dst || bytes < 16 || (bytes & 15) || grid <= 0 || variant < 0 || variant > 7) return -1;
  clear_errors();
  hipStream_t st = static_cast<hipStream_t>(stream);
  u32x4* d = static_cast<u32x4*>(dst);
  const int64_t n = bytes >> 4;
  switch (variant) {
    case 0: write_var_kernel<false, 1, false><<<grid, 256, 0, st>>>(d, n); break;
    case 1: write_var_kernel<true, 1, false><<<grid, 256, 0, st>>>(d, n); break;
    case 2: write_var_kernel<false, 2, false><<<grid, 256, 0, st>>>(d, n); break;
    case 3: write_var_kernel<true, 2, false><<<grid, 256, 0, st>>>(d, n); break;
    case 4: write_var_kernel<false, 1, true><<<grid, 256, 0, st>>>(d, n); break;
    case 5: write_var_kernel<true, 1, true><<<grid, 256, 0, st>>>(d, n); break;
    case 6: write_var_kernel<false, 2, true><<<grid, 256, 0, st>>>(d, n); break;
    default: write_var_kernel<true, 2, true><<<grid, 256, 0, st>>>(d, n); break;
  }
  return launched();
}

int rkvc_copy_var(const void* src, void* dst, int64_t bytes, int grid, int variant,
                  void* stream) {
  if (!src || !dst || bytes < 16 || (bytes & 15) || grid <= 0 || variant < 0 || variant > 15)
    return -1;
  clear_errors();
  hipStream_t st = static_cast<hipStream_t>(stream);
  const u32x4* s = static_cast<const u32x4*>(src);
  u32x4* d = static_cast<u32x4*>(dst);
  const int64_t n = bytes >> 4;
#define RKVC_COPY(V, NTL, NTS, VPL, CH) \
  case V: copy_var_kernel<NTL, NTS, VPL, CH><<<grid, 256, 0, st>>>(s, d, n); break;
  switch (variant) {
    RKVC_COPY(0, false, false, 1, false) RKVC_COPY(1, false, true, 1, false)
    RKVC_COPY(2, false, false, 2, false) RKVC_COPY(3, false, true, 2, false)
    RKVC_COPY(4, false, false, 1, true) RKVC_COPY(5, false, true, 1, true)
    RKVC_COPY(6, false, false, 2, true) RKVC_COPY(7, false, true, 2, true)
    RKVC_COPY(8, true, false, 1, false) RKVC_COPY(9, true, true, 1, false)
    RKVC_COPY(10, true, false, 2, false) RKVC_COPY(11, true, true, 2, false)
    RKVC_COPY(12, true, false, 1, true) RKVC_COPY(13, true, true, 1, true)
    RKVC_COPY(14, true, false, 2, true) default: copy_var_kernel<true, true, 2, true>
        <<<grid, 256, 0, st>>>(s, d, n); break;
  }
#undef RKVC_COPY
  return launched();
}

int rkvc_block_copy_pipe(void* pool, const int32_t* pairs, int n_pairs, int64_t num_blocks,
                         int grid, void* stream) {
  if (!pool || !pairs || n_pairs <= 0 || num_blocks <= 0 || grid <= 0) return -1;
  clear_errors();
  block_copy_pipe_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<char*>(pool), pairs, n_pairs, num_blocks);
  return launched();
}

// unr in {1, 2, 4, 8}; grid 0: one round per workgroup.  copy: nt stores when
// variant & 1.
int rkvc_write_unr(void* dst, int64_t bytes, int unr, int grid, void* stream) {
  if (!dst || bytes < 16 || (bytes & 15) || grid < 0) return -1;
  const int64_t n = bytes >> 4;
  const int64_t g = grid ? grid : (n + 256 * unr - 1) / (256 * unr);
  if (g > INT32_MAX) return -1;
  clear_errors();
  hipStream_t st = static_cast<hipStream_t>(stream);
  u32x4* d = static_cast<u32x4*>(dst);
  switch (unr) {
    case 1: write_unr_kernel<1><<<(unsigned)g, 256, 0, st>>>(d, n); break;
    case 2: write_unr_kernel<2><<<(unsigned)g, 256, 0, st>>>(d, n); break;
    case 4: write_unr_kernel<4><<<(unsigned)g, 256, 0, st>>>(d, n); break;
    case 8: write_unr_kernel<8><<<(unsigned)g, 256, 0, st>>>(d, n); break;
    default: return -1;
  }
  return launched();
}

int rkvc_read_unr(const void* src, int64_t bytes, unsigned* sink, unsigned magic, int unr,
                  int grid, void* stream) {
  if (!src || !sink || bytes < 16 || (bytes & 15) || grid < 0) return -1;
  const int64_t n = bytes >> 4;
  const int64_t g = grid ? grid : (n + 256 * unr - 1) / (256 * unr);
  if (g > INT32_MAX) return -1;
  clear_errors();
  hipStream_t st = static_cast<hipStream_t>(stream);
  const u32x4* s = static_cast<const u32x4*>(src);
  switch (unr) {
    case 1: read_unr_kernel<1><<<(unsigned)g, 256, 0, st>>>(s, n, sink, magic); break;
    case 2: read_unr_kernel<2><<<(unsigned)g, 256, 0, st>>>(s, n, sink, magic); break;
    case 4: read_unr_kernel<4><<<(unsigned)g, 256, 0, st>>>(s, n, sink, magic); break;
    case 8: read_unr_kernel<8><<<(unsigned)g, 256, 0, st>>>(s, n, sink, magic); break;
    case 16: read_unr_kernel<16><<<(unsigned)g, 256, 0, st>>>(s, n, sink, magic); break;
    default: return -1;
  }
  return launched();
}

int rkvc_copy_unr(const void* src, void* dst, int64_t bytes, int unr, int grid, int nt,
                  void* stream) {
  if (!src || !dst || bytes < 16 || (bytes & 15) || grid < 0) return -1;
  const int64_t n = bytes >> 4;
  const int64_t g = grid ? grid : (n + 256 * unr - 1) / (256 * unr);
  if (g > INT32_MAX) return -1;
  clear_errors();
  hipStream_t st = static_cast<hipStream_t>(stream);
  const u32x4* s = static_cast<const u32x4*>(src);
  u32x4* d = static_cast<u32x4*>(dst);
#define RKVC_CU(U) \
  case U: \
    if (nt) copy_unr_kernel<U, true><<<(unsigned)g, 256, 0, st>>>(s, d, n); \
    else copy_unr_kernel<U, false><<<(unsigned)g, 256, 0, st>>>(s, d, n); \
    break;
  switch (unr) {
    RKVC_CU(1) RKVC_CU(2) RKVC_CU(4) RKVC_CU(8)
    default: return -1;
  }
#undef RKVC_CU
  return launched();
}

// block_bytes a multiple of 4096 * unr.
int rkvc_block_copy_unr(void* pool, const int32_t* pairs, int n_pairs, int64_t block_bytes,
                        int64_t num_blocks, int unr, void* stream) {
  if (!pool || !pairs || n_pairs <= 0 || n_pairs > 65535 || block_bytes <= 0 ||
      num_blocks <= 0 || (unr != 1 && unr != 2 && unr != 4 && unr != 8) ||
      block_bytes % (4096 * unr))
    return -1;
  clear_errors();
  const dim3 grid((unsigned)(block_bytes / (4096 * unr)), (unsigned)n_pairs);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* p = static_cast<char*>(pool);
  switch (unr) {
    case 1: block_copy_unr_kernel<1><<<grid, 256, 0, st>>>(p, pairs, block_bytes, num_blocks); break;
    case 2: block_copy_unr_kernel<2><<<grid, 256, 0, st>>>(p, pairs, block_bytes, num_blocks); break;
    case 4: block_copy_unr_kernel<4><<<grid, 256, 0, st>>>(p, pairs, block_bytes, num_blocks); break;
    default: block_copy_unr_kernel<8><<<grid, 256, 0, st>>>(p, pairs, block_bytes, num_blocks); break;
  }
  return launched();
}

// kind 0: write `bytes` of dst; 1: copy `bytes` from src to dst; 2: block
// copies of the n_pairs pairs of block_bytes-byte blocks inside dst (src
// unused); nth threads (64, 128, 256 or 512) and 16 nth bytes a workgroup.
int rkvc_nth(int kind, const void* src, void* dst, int64_t bytes, const int32_t* pairs,
             int n_pairs, int64_t block_bytes, int64_t num_blocks, int nth, void* stream) {
  if (!dst || (nth != 64 && nth != 128 && nth != 256 && nth != 512) || kind < 0 || kind > 2)
    return -1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid;
  int64_t n = 0;
  if (kind < 2) {
    if (bytes < 16 || (bytes & 15) || (kind == 1 && !src)) return -1;
    n = bytes >> 4;
    const int64_t g = (n + nth - 1) / nth;
    if (g > INT32_MAX) return -1;
    grid = dim3((unsigned)g);
  } else {
    if (!pairs || n_pairs <= 0 || n_pairs > 65535 || block_bytes <= 0 || num_blocks <= 0 ||
        block_bytes % (16 * nth))
      return -1;
    grid = dim3((unsigned)(block_bytes / (16 * nth)), (unsigned)n_pairs);
  }
  clear_errors();
  u32x4* d = static_cast<u32x4*>(dst);
  const u32x4* s = static_cast<const u32x4*>(src);
  char* p = static_cast<char*>(dst);
#define RKVC_NTH(T)                                                                           \
  case T:                                                                                     \
    if (kind == 0) write_nth_kernel<T><<<grid, T, 0, st>>>(d, n);                             \
    else if (kind == 1) copy_nth_kernel<T><<<grid, T, 0, st>>>(s, d, n);                      \
    else block_copy_nth_kernel<T><<<grid, T, 0, st>>>(p, pairs, block_bytes, num_blocks);    \
    break;
  switch (nth) {
    RKVC_NTH(64) RKVC_NTH(128) RKVC_NTH(256) RKVC_NTH(512)
  }
#undef RKVC_NTH
  return launched();
}

int rkvc_block_copy(void* pool, const int32_t* pairs, int n_pairs, int64_t block_bytes,
                    int64_t num_blocks, void* stream) {
  if (!pool || !pairs || n_pairs <= 0 || block_bytes <= 0 || (block_bytes & 15) ||
      num_blocks <= 0)
    return -1;
  clear_errors();
  block_copy_kernel<<<n_pairs, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<char*>(pool), pairs, block_bytes, num_blocks);
  return launched();
}

// Pools [num_blocks][num_kv_heads][16][128] of elem_bytes-byte elements
// (2: bf16; 1: int8 / fp8, with fp32 scales [num_blocks][num_kv_heads][16]);
// tables int32 [B][max_blocks] (ids outside [0, num_blocks) are absent);
// partitions = ceil(max_ctx / 640).
int rkvc_tile_stream(const void* k_pool, const void* v_pool, const float* k_scale,
                     const float* v_scale, int elem_bytes, const int32_t* tables, int max_blocks,
                     const int32_t* ctx_lens, int num_seqs, int num_kv_heads, int64_t num_blocks,
                     int partitions, unsigned* sink, unsigned magic, void* stream) {
  if (!k_pool || !v_pool || !tables || !ctx_lens || !sink || max_blocks <= 0 ||
      num_seqs <= 0 || num_kv_heads <= 0 || num_blocks <= 0 || partitions <= 0 ||
      (elem_bytes != 1 && elem_bytes != 2) || (elem_bytes == 1 && (!k_scale || !v_scale)))
    return -1;
  const dim3 grid((unsigned)num_kv_heads, (unsigned)partitions, (unsigned)num_seqs);
  clear_errors();
  auto kern = elem_bytes == 2 ? tile_stream_kernel<2> : tile_stream_kernel<1>;
  kern<<<grid, 64 * kSplit, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint8_t*>(k_pool), static_cast<const uint8_t*>(v_pool), k_scale, v_scale,
      tables, max_blocks, ctx_lens, num_kv_heads, num_blocks, sink, magic);
  return launched();
}

// The bf16 decode pattern at the partition shapes of the decode kernel's
// builds: (tiles a wave, waves a workgroup) = (10, 4) 640 tokens, (6, 8)
// 768, (10, 8) 1280; grid (Hkv, partitions, sequences) as rkvc_tile_stream.
int rkvc_tile_stream_shape(const void* k_pool, const void* v_pool, const int32_t* tables,
                           int max_blocks, const int32_t* ctx_lens, int num_seqs,
                           int num_kv_heads, int64_t num_blocks, int partitions, int ntw,
                           int split, unsigned* sink, unsigned magic, void* stream) {
  if (!k_pool || !v_pool || !tables || !ctx_lens || !sink || max_blocks <= 0 || num_seqs <= 0 ||
      num_kv_heads <= 0 || num_blocks <= 0 || partitions <= 0)
    return -1;
  auto kern = ntw == 10 && split == 4   ? tile_stream_kernel<2, 10, 4>
              : ntw == 6 && split == 8  ? tile_stream_kernel<2, 6, 8>
              : ntw == 10 && split == 8 ? tile_stream_kernel<2, 10, 8>
                                        : nullptr;
  if (!kern) return -1;
  const dim3 grid((unsigned)num_kv_heads, (unsigned)partitions, (unsigned)num_seqs);
  clear_errors();
  kern<<<grid, 64 * split, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint8_t*>(k_pool), static_cast<const uint8_t*>(v_pool), nullptr, nullptr,
      tables, max_blocks, ctx_lens, num_kv_heads, num_blocks, sink, magic);
  return launched();
}

// variant: 0 the decode pattern (row scales), 1 no scales, 2 two KV heads per
// wave, 3 four, 4 partition-major grid, 5 scales after each K tile (k_pool
// of num_blocks * Hkv tiles of 2,176 bytes; k_scale / v_scale unused).
int rkvc_tile_stream_1b(const void* k_pool, const void* v_pool, const float* k_scale,
                        const float* v_scale, const int32_t* tables, int max_blocks,
                        const int32_t* ctx_lens, int num_seqs, int num_kv_heads,
                        int64_t num_blocks, int partitions, int variant, unsigned* sink,
                        unsigned magic, void* stream) {
  const int hpw = variant == 2 ? 2 : variant == 3 ? 4 : 1;
  const bool scales = variant == 0 || variant == 2 || variant == 3 || variant == 4;
  if (!k_pool || !v_pool || !tables || !ctx_lens || !sink || max_blocks <= 0 || num_seqs <= 0 ||
      num_kv_heads <= 0 || num_blocks <= 0 || partitions <= 0 || variant < 0 || variant > 5 ||
      num_kv_heads % hpw || (scales && (!k_scale || !v_scale)))
    return -1;
  const unsigned hx = (unsigned)(num_kv_heads / hpw);
  const dim3 grid = variant == 4 ? dim3(hx, (unsigned)num_seqs, (unsigned)partitions)
                                 : dim3(hx, (unsigned)partitions, (unsigned)num_seqs);
  auto kern = variant == 0 ? tile_stream1_kernel<1, 1, false>
            : variant == 1 ? tile_stream1_kernel<1, 0, false>
            : variant == 2 ? tile_stream1_kernel<2, 1, false>
            : variant == 3 ? tile_stream1_kernel<4, 1, false>
            : variant == 4 ? tile_stream1_kernel<1, 1, true>
                           : tile_stream1_kernel<1, 2, false>;
  clear_errors();
  kern<<<grid, 64 * kSplit, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint8_t*>(k_pool), static_cast<const uint8_t*>(v_pool), k_scale, v_scale,
      tables, max_blocks, ctx_lens, num_kv_heads, num_blocks, sink, magic);
  return launched();
}

}  // extern "C"
