// paged_decode.hip -- single-token paged decode attention with GQA, split-K,
// for gfx950 (CDNA4, wave64).
//
// Pass 1 (decode_partition_kernel): one workgroup per (partition of P tokens,
// KV head, sequence).  The G = Hq/Hkv query heads that share a KV head are
// served by the same workgroup, so every K/V byte is read from HBM once.
//   * Lane mapping: a wave reads one (block, head) tile [BS][D] as NL
//     coalesced 1 KiB loads: lane l takes 16 bytes of token row l / LPT at
//     dims (l % LPT) * E ... + E, where E = 16 / sizeof(elem) and
//     LPT = D / E lanes cover one row.
//   * QK^T: each lane multiplies its E key elements with the matching E
//     elements of the G (pre-scaled) queries held in registers, then a DPP
//     sum over the LPT lanes of the row gives the G scores of that token.
//   * Scores go to LDS; the workgroup takes the max and the sum of
//     exp2(s - max) over the partition (two-pass softmax inside the
//     partition: no running rescale of the accumulators).
//   * PV: the same lane mapping over V; each lane accumulates
//     p[g][token] * v for its E dims, then lanes of different rows and
//     different waves are summed (shuffles + LDS).
//   * All K and V loads of a wave's tiles are issued before any math, so a
//     wave keeps TPW * NL * 2 16-byte loads in flight.
// Pass 2 (decode_merge_kernel): per (query head, sequence) merge of the
// partition partials m (max), l (sum), acc (unnormalised PV):
//   M = max m_p;  out = sum_p 2^(m_p - M) acc_p / sum_p 2^(m_p - M) l_p.
// Sequences that fit one partition are finished in pass 1.
//
// Scores are kept in the log2 domain: q is pre-multiplied by
// scale * log2(e), so softmax uses exp2 (v_exp_f32) directly.
#include "common.hpp"

#include <cmath>

namespace rkv {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

template <typename T>
struct Traits;
template <>
struct Traits<float> {
  static constexpr int E = 4;
};
template <>
struct Traits<uint16_t> {
  static constexpr int E = 8;
};

// Converts one 16-byte load into E floats.
__device__ __forceinline__ void to_float(const uint4& w, float (&f)[8]) {
  f[0] = bf16_lo(w.x);
  f[1] = bf16_hi(w.x);
  f[2] = bf16_lo(w.y);
  f[3] = bf16_hi(w.y);
  f[4] = bf16_lo(w.z);
  f[5] = bf16_hi(w.z);
  f[6] = bf16_lo(w.w);
  f[7] = bf16_hi(w.w);
}
__device__ __forceinline__ void to_float(const uint4& w, float (&f)[4]) {
  f[0] = __uint_as_float(w.x);
  f[1] = __uint_as_float(w.y);
  f[2] = __uint_as_float(w.z);
  f[3] = __uint_as_float(w.w);
}

template <typename T, int D, int G, int BS, int NW, int TPW>
__global__ __launch_bounds__(NW * 64) void decode_partition_kernel(
    float* __restrict__ out, float* __restrict__ part_acc, float* __restrict__ part_ml,
    const float* __restrict__ q, const void* __restrict__ k_pool_,
    const void* __restrict__ v_pool_, const int32_t* __restrict__ block_tables,
    int max_blocks_per_seq, const int32_t* __restrict__ ctx_lens, int ctx_cap, int num_kv_heads,
    int64_t num_blocks, float q_scale, int max_parts) {
  const T* __restrict__ k_pool = static_cast<const T*>(k_pool_);
  const T* __restrict__ v_pool = static_cast<const T*>(v_pool_);
  constexpr int E = Traits<T>::E;
  constexpr int LPT = D / E;     // lanes per token row
  constexpr int TPL = 64 / LPT;  // token rows per wave-load
  constexpr int NL = BS / TPL;   // wave-loads per (block, head) tile
  constexpr int P = TPW * NW * BS;
  constexpr int NT = NW * 64;
  static_assert(D % E == 0 && 64 % LPT == 0 && BS % TPL == 0, "unsupported tile shape");

  __shared__ __align__(16) float s_p[P * G];  // scores, then probabilities [token][g]
  __shared__ float s_red[NW][G];
  __shared__ float s_m[G], s_l[G];
  __shared__ __align__(16) float s_acc[NW][G * D];

  const int part = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
  const int num_q_heads = num_kv_heads * G;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slot = lane / LPT, dl = lane % LPT;

  int L = ctx_lens[b];
  L = L < 0 ? 0 : (L > ctx_cap ? ctx_cap : L);
  const int nparts = (L + P - 1) / P;
  const int64_t head0 = (int64_t)b * num_q_heads + kh * G;  // first query head row
  if (L == 0) {
    if (part == 0)
      for (int o = tid; o < G * D; o += NT) out[head0 * D + o] = 0.0f;
    return;
  }
  if (part >= nparts) return;

  // ---- issue every K and V load of this wave ----
  uint4 kr[TPW][NL], vr[TPW][NL];
  bool tile_ok[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int lb = part * (P / BS) + w + NW * i;  // logical block of the sequence
    const int tbase = lb * BS;
    int32_t pb = -1;
    if (tbase < L) pb = block_tables[(int64_t)b * max_blocks_per_seq + lb];
    const bool ok = (tbase < L) && pb >= 0 && pb < num_blocks;
    tile_ok[i] = ok;
    const int64_t base = ((int64_t)(ok ? pb : 0) * num_kv_heads + kh) * BS * D + dl * E;
#pragma unroll
    for (int n = 0; n < NL; ++n) {
      const int row = n * TPL + slot;
      if (ok && tbase + row < L) {
        kr[i][n] = *reinterpret_cast<const uint4*>(k_pool + base + row * D);
        vr[i][n] = *reinterpret_cast<const uint4*>(v_pool + base + row * D);
      } else {
        kr[i][n] = make_uint4(0, 0, 0, 0);
        vr[i][n] = make_uint4(0, 0, 0, 0);
      }
    }
  }

  // ---- queries, pre-scaled into the exp2 domain ----
  float qf[G][E];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float* qp = q + (head0 + g) * D + dl * E;
#pragma unroll
    for (int e = 0; e < E; e += 4) {
      const float4 v = *reinterpret_cast<const float4*>(qp + e);
      qf[g][e + 0] = v.x * q_scale;
      qf[g][e + 1] = v.y * q_scale;
      qf[g][e + 2] = v.z * q_scale;
      qf[g][e + 3] = v.w * q_scale;
    }
  }

  // ---- phase 1: scores ----
  const int tok0 = part * P;
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
#pragma unroll
    for (int n = 0; n < NL; ++n) {
      float kf[E];
      to_float(kr[i][n], kf);
      float s[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float a = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) a = fmaf(qf[g][e], kf[e], a);
        s[g] = group_sum<LPT>(a);
      }
      const int tp = (w + NW * i) * BS + n * TPL + slot;  // token within the partition
      const bool valid = tile_ok[i] && (tok0 + tp < L);
      if (dl == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) s_p[tp * G + g] = valid ? s[g] : -INFINITY;
      }
    }
  }
  __syncthreads();

  // ---- softmax statistics over the partition ----
  {
    float mloc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) mloc[g] = -INFINITY;
    for (int t = tid; t < P; t += NT)
#pragma unroll
      for (int g = 0; g < G; ++g) mloc[g] = fmaxf(mloc[g], s_p[t * G + g]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      mloc[g] = wave_max(mloc[g]);
      if (lane == 0) s_red[w][g] = mloc[g];
    }
    __syncthreads();
    float m[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = s_red[0][g];
#pragma unroll
      for (int x = 1; x < NW; ++x) m[g] = fmaxf(m[g], s_red[x][g]);
    }
    __syncthreads();
    float lloc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) lloc[g] = 0.0f;
    for (int t = tid; t < P; t += NT)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float s = s_p[t * G + g];
        const float p = (s == -INFINITY) ? 0.0f : exp2f(s - m[g]);
        s_p[t * G + g] = p;
        lloc[g] += p;
      }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      lloc[g] = wave_sum(lloc[g]);
      if (lane == 0) s_red[w][g] = lloc[g];
    }
    __syncthreads();
    if (tid == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float l = 0.0f;
#pragma unroll
        for (int x = 0; x < NW; ++x) l += s_red[x][g];
        s_m[g] = m[g];
        s_l[g] = l;
      }
    }
  }

  // ---- phase 2: PV ----
  float acc[G][E];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < E; ++e) acc[g][e] = 0.0f;
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
#pragma unroll
    for (int n = 0; n < NL; ++n) {
      float vf[E];
      to_float(vr[i][n], vf);
      const int tp = (w + NW * i) * BS + n * TPL + slot;
      float p[G];
#pragma unroll
      for (int g = 0; g < G; ++g) p[g] = s_p[tp * G + g];
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[g][e] = fmaf(p[g], vf[e], acc[g][e]);
    }
  }
  // sum over the TPL token rows of the wave
#pragma unroll
  for (int o = LPT; o < 64; o <<= 1)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < E; ++e) acc[g][e] += __shfl_xor(acc[g][e], o);
  if (slot == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < E; e += 4)
        *reinterpret_cast<float4*>(&s_acc[w][g * D + dl * E + e]) =
            make_float4(acc[g][e], acc[g][e + 1], acc[g][e + 2], acc[g][e + 3]);
  }
  __syncthreads();

  // ---- sum over waves, then finish or emit a partial ----
  for (int o = tid; o < G * D; o += NT) {
    float v = 0.0f;
#pragma unroll
    for (int x = 0; x < NW; ++x) v += s_acc[x][o];
    const int g = o / D, d = o - g * D;
    const float l = s_l[g];
    if (nparts == 1) {
      out[(head0 + g) * D + d] = l > 0.0f ? v / l : 0.0f;
    } else {
      const int64_t row = (head0 + g) * max_parts + part;
      part_acc[row * D + d] = v;
      if (d == 0) {
        part_ml[row * 2 + 0] = s_m[g];
        part_ml[row * 2 + 1] = l;
      }
    }
  }
}

// grid = (num_q_heads, num_seqs), D threads (>= 64).
template <int D>
__global__ __launch_bounds__(D < 64 ? 64 : D) void decode_merge_kernel(
    float* __restrict__ out, const float* __restrict__ part_acc,
    const float* __restrict__ part_ml, const int32_t* __restrict__ ctx_lens, int ctx_cap,
    int num_q_heads, int P, int max_parts) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  int L = ctx_lens[b];
  L = L < 0 ? 0 : (L > ctx_cap ? ctx_cap : L);
  const int np = (L + P - 1) / P;
  if (np <= 1 || d >= D) return;
  const int64_t row0 = ((int64_t)b * num_q_heads + h) * max_parts;
  float M = -INFINITY;
  for (int p = 0; p < np; ++p) M = fmaxf(M, part_ml[(row0 + p) * 2]);
  float num = 0.0f, den = 0.0f;
  if (M != -INFINITY) {
    for (int p = 0; p < np; ++p) {
      const float m = part_ml[(row0 + p) * 2];
      const float wgt = (m == -INFINITY) ? 0.0f : exp2f(m - M);
      den = fmaf(wgt, part_ml[(row0 + p) * 2 + 1], den);
      num = fmaf(wgt, part_acc[(row0 + p) * D + d], num);
    }
  }
  out[((int64_t)b * num_q_heads + h) * D + d] = den > 0.0f ? num / den : 0.0f;
}

// ---- dispatch ----------------------------------------------------------------

constexpr int kBS = 16;
constexpr int kP = 256;  // tokens per partition

struct Launch {
  int nw = 0;
  void (*kernel)(float*, float*, float*, const float*, const void*, const void*, const int32_t*,
                 int, const int32_t*, int, int, int64_t, float, int) = nullptr;
};

template <typename T, int D, int G, int NW>
Launch make_launch() {
  constexpr int TPW = kP / (NW * kBS);
  Launch l;
  l.nw = NW;
  l.kernel = &decode_partition_kernel<T, D, G, kBS, NW, TPW>;
  return l;
}

// (T, D) -> waves per workgroup; tiles per wave = kP / (NW * 16).  Chosen so
// a wave holds at most 16 16-byte K+V loads per lane (64 VGPRs each of K, V).
template <typename T, int D>
constexpr int waves_for() {
  return (sizeof(T) == 4 && D == 128) ? 8 : 4;
}

template <typename T, int D>
Launch pick_g(int G) {
  constexpr int NW = waves_for<T, D>();
  switch (G) {
    case 1: return make_launch<T, D, 1, NW>();
    case 2: return make_launch<T, D, 2, NW>();
    case 4: return make_launch<T, D, 4, NW>();
    case 8: return make_launch<T, D, 8, NW>();
    default: return Launch{};
  }
}

template <typename T>
Launch pick_d(int D, int G) {
  switch (D) {
    case 32: return pick_g<T, 32>(G);
    case 64: return pick_g<T, 64>(G);
    case 128: return pick_g<T, 128>(G);
    default: return Launch{};
  }
}

struct DecodeArgs {
  float* out;
  const float* q;
  const void* k_pool;
  const void* v_pool;
  const int32_t* block_tables;
  int max_blocks_per_seq;
  const int32_t* ctx_lens;
  int num_seqs, num_q_heads, num_kv_heads, head_dim, block_size;
  int64_t num_blocks;
  int max_context;
  float scale;
  int dtype, partition_size;
  void* workspace;
  size_t workspace_bytes;
  hipStream_t stream;
};

size_t ws_bytes(int B, int Hq, int D, int max_parts) {
  if (max_parts <= 1) return 0;
  const size_t rows = (size_t)B * Hq * max_parts;
  const size_t acc = rows * D * sizeof(float);
  const size_t acc_pad = (acc + 255) & ~size_t(255);
  return acc_pad + rows * 2 * sizeof(float);
}

int ctx_cap_of(int max_context, int max_blocks_per_seq, int block_size) {
  const int64_t cap = (int64_t)max_blocks_per_seq * block_size;
  return (int)(max_context < cap ? max_context : cap);
}

int validate(const DecodeArgs& a, int& max_parts) {
  if (a.num_seqs < 0 || a.max_blocks_per_seq < 0 || a.num_blocks < 0)
    return fail(RKV_ERR_INVALID_ARG, "negative size argument");
  if (a.num_q_heads <= 0 || a.num_kv_heads <= 0 || a.num_q_heads % a.num_kv_heads)
    return fail(RKV_ERR_INVALID_ARG, "num_q_heads must be a positive multiple of num_kv_heads");
  if (a.dtype != RKV_F32 && a.dtype != RKV_BF16)
    return fail(RKV_ERR_INVALID_ARG, "dtype must be RKV_F32 or RKV_BF16");
  if (a.block_size != kBS) return fail(RKV_ERR_UNSUPPORTED, "block_size must be 16");
  if (a.head_dim != 32 && a.head_dim != 64 && a.head_dim != 128)
    return fail(RKV_ERR_UNSUPPORTED, "head_dim must be 32, 64 or 128");
  const int G = a.num_q_heads / a.num_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return fail(RKV_ERR_UNSUPPORTED, "num_q_heads / num_kv_heads must be 1, 2, 4 or 8");
  if (a.partition_size > 0 && a.partition_size != kP)
    return fail(RKV_ERR_UNSUPPORTED, "partition_size must be 256 (or <= 0 for the default)");
  if (a.num_seqs > 65535 || a.num_kv_heads > 65535)
    return fail(RKV_ERR_INVALID_ARG, "num_seqs and num_kv_heads must be <= 65535");
  if (a.max_context < 0) return fail(RKV_ERR_INVALID_ARG, "max_context must be >= 0");
  const int cap = ctx_cap_of(a.max_context, a.max_blocks_per_seq, a.block_size);
  max_parts = cap <= 0 ? 1 : (cap + kP - 1) / kP;
  if (a.num_seqs == 0) return RKV_OK;
  if (!a.out || !a.q || !a.k_pool || !a.v_pool || !a.block_tables || !a.ctx_lens)
    return fail(RKV_ERR_INVALID_ARG, "null pointer argument");
  if (!aligned16(a.out) || !aligned16(a.q) || !aligned16(a.k_pool) || !aligned16(a.v_pool))
    return fail(RKV_ERR_INVALID_ARG, "out, q and pools must be 16-byte aligned");
  const size_t need = ws_bytes(a.num_seqs, a.num_q_heads, a.head_dim, max_parts);
  if (need > 0 && (!a.workspace || a.workspace_bytes < need))
    return fail(RKV_ERR_WORKSPACE, "workspace missing or smaller than rkv_decode_workspace_bytes()");
  if (need > 0 && !aligned16(a.workspace))
    return fail(RKV_ERR_INVALID_ARG, "workspace must be 16-byte aligned");
  return RKV_OK;
}

void split_ws(void* ws, int B, int Hq, int D, int max_parts, float*& acc, float*& ml) {
  const size_t rows = (size_t)B * Hq * max_parts;
  const size_t acc_pad = (rows * D * sizeof(float) + 255) & ~size_t(255);
  acc = static_cast<float*>(ws);
  ml = reinterpret_cast<float*>(static_cast<char*>(ws) + acc_pad);
}

int launch_partitions(const DecodeArgs& a, int max_parts) {
  const int G = a.num_q_heads / a.num_kv_heads;
  Launch l = a.dtype == RKV_BF16 ? pick_d<uint16_t>(a.head_dim, G) : pick_d<float>(a.head_dim, G);
  if (!l.kernel) return fail(RKV_ERR_UNSUPPORTED, "no decode kernel for this shape");
  float *acc = nullptr, *ml = nullptr;
  if (max_parts > 1) split_ws(a.workspace, a.num_seqs, a.num_q_heads, a.head_dim, max_parts, acc, ml);
  const int cap = ctx_cap_of(a.max_context, a.max_blocks_per_seq, a.block_size);
  dim3 grid((unsigned)max_parts, (unsigned)a.num_kv_heads, (unsigned)a.num_seqs);
  hipLaunchKernelGGL(l.kernel, grid, dim3(l.nw * 64), 0, a.stream, a.out, acc, ml, a.q, a.k_pool,
                     a.v_pool, a.block_tables, a.max_blocks_per_seq, a.ctx_lens, cap,
                     a.num_kv_heads, a.num_blocks, a.scale * kLog2e, max_parts);
  return check_launch("decode_partition_kernel");
}

int launch_merge(float* out, const int32_t* ctx_lens, int num_seqs, int num_q_heads, int head_dim,
                 int cap, int max_parts, void* ws, hipStream_t stream) {
  if (max_parts <= 1 || num_seqs == 0) return RKV_OK;
  float *acc = nullptr, *ml = nullptr;
  split_ws(ws, num_seqs, num_q_heads, head_dim, max_parts, acc, ml);
  dim3 grid((unsigned)num_q_heads, (unsigned)num_seqs);
  switch (head_dim) {
    case 32:
      decode_merge_kernel<32><<<grid, 64, 0, stream>>>(out, acc, ml, ctx_lens, cap, num_q_heads,
                                                       kP, max_parts);
      break;
    case 64:
      decode_merge_kernel<64><<<grid, 64, 0, stream>>>(out, acc, ml, ctx_lens, cap, num_q_heads,
                                                       kP, max_parts);
      break;
    default:
      decode_merge_kernel<128><<<grid, 128, 0, stream>>>(out, acc, ml, ctx_lens, cap,
                                                         num_q_heads, kP, max_parts);
      break;
  }
  return check_launch("decode_merge_kernel");
}

}  // namespace
}  // namespace rkv

using namespace rkv;

extern "C" size_t rkv_decode_workspace_bytes(int num_seqs, int num_q_heads, int head_dim,
                                             int max_context, int partition_size) {
  (void)partition_size;
  if (num_seqs <= 0 || num_q_heads <= 0 || head_dim <= 0 || max_context <= 0) return 0;
  const int max_parts = (max_context + kP - 1) / kP;
  return ws_bytes(num_seqs, num_q_heads, head_dim, max_parts);
}

extern "C" int rkv_decode_partition_size(int partition_size, int head_dim, int dtype) {
  (void)partition_size;
  (void)head_dim;
  (void)dtype;
  return kP;
}

extern "C" int rkv_decode_attention_partitions(
    float* out, const float* q, const void* k_pool, const void* v_pool,
    const int32_t* block_tables, int max_blocks_per_seq, const int32_t* ctx_lens, int num_seqs,
    int num_q_heads, int num_kv_heads, int head_dim, int block_size, int64_t num_blocks,
    int max_context, float scale, int dtype, int partition_size, void* workspace,
    size_t workspace_bytes, void* stream) {
  clear_error();
  DecodeArgs a{out, q, k_pool, v_pool, block_tables, max_blocks_per_seq, ctx_lens, num_seqs,
               num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, max_context, scale,
               dtype, partition_size, workspace, workspace_bytes,
               static_cast<hipStream_t>(stream)};
  int max_parts = 1;
  if (int rc = validate(a, max_parts)) return rc;
  if (num_seqs == 0) return RKV_OK;
  return launch_partitions(a, max_parts);
}

extern "C" int rkv_decode_attention_merge(float* out, const int32_t* ctx_lens,
                                          int max_blocks_per_seq, int num_seqs, int num_q_heads,
                                          int head_dim, int block_size, int max_context,
                                          int dtype, int partition_size, const void* workspace,
                                          size_t workspace_bytes, void* stream) {
  clear_error();
  (void)dtype;
  if (num_seqs < 0 || num_q_heads <= 0 || max_blocks_per_seq < 0 || max_context < 0)
    return fail(RKV_ERR_INVALID_ARG, "bad size argument");
  if (block_size != kBS) return fail(RKV_ERR_UNSUPPORTED, "block_size must be 16");
  if (head_dim != 32 && head_dim != 64 && head_dim != 128)
    return fail(RKV_ERR_UNSUPPORTED, "head_dim must be 32, 64 or 128");
  if (partition_size > 0 && partition_size != kP)
    return fail(RKV_ERR_UNSUPPORTED, "partition_size must be 256 (or <= 0 for the default)");
  if (num_seqs > 65535 || num_q_heads > 65535)
    return fail(RKV_ERR_INVALID_ARG, "num_seqs and num_q_heads must be <= 65535");
  const int cap = ctx_cap_of(max_context, max_blocks_per_seq, block_size);
  const int max_parts = cap <= 0 ? 1 : (cap + kP - 1) / kP;
  if (max_parts <= 1 || num_seqs == 0) return RKV_OK;
  if (!out || !ctx_lens) return fail(RKV_ERR_INVALID_ARG, "null pointer argument");
  const size_t need = ws_bytes(num_seqs, num_q_heads, head_dim, max_parts);
  if (!workspace || workspace_bytes < need)
    return fail(RKV_ERR_WORKSPACE, "workspace missing or smaller than rkv_decode_workspace_bytes()");
  return launch_merge(out, ctx_lens, num_seqs, num_q_heads, head_dim, cap, max_parts,
                      const_cast<void*>(workspace), static_cast<hipStream_t>(stream));
}

extern "C" int rkv_decode_attention(float* out, const float* q, const void* k_pool,
                                    const void* v_pool, const int32_t* block_tables,
                                    int max_blocks_per_seq, const int32_t* ctx_lens, int num_seqs,
                                    int num_q_heads, int num_kv_heads, int head_dim,
                                    int block_size, int64_t num_blocks, int max_context,
                                    float scale, int dtype, int partition_size, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  int rc = rkv_decode_attention_partitions(out, q, k_pool, v_pool, block_tables,
                                           max_blocks_per_seq, ctx_lens, num_seqs, num_q_heads,
                                           num_kv_heads, head_dim, block_size, num_blocks,
                                           max_context, scale, dtype, partition_size, workspace,
                                           workspace_bytes, stream);
  if (rc) return rc;
  return rkv_decode_attention_merge(out, ctx_lens, max_blocks_per_seq, num_seqs, num_q_heads,
                                    head_dim, block_size, max_context, dtype, partition_size,
                                    workspace, workspace_bytes, stream);
}
