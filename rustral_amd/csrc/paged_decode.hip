// paged_decode.hip -- single-token paged decode attention with GQA, split-K,
// for gfx950 (CDNA4, wave64).
//
// Pass 1 (decode_stream_kernel) splits every sequence into partitions of P
// tokens and produces, per (partition, query head), the partial softmax state
// (m, l, acc); the G = Hq/Hkv query heads that share a KV head are served by
// the same workgroup, so every K/V byte is read from HBM once.  SPLIT waves
// per (partition, KV head, sequence) each stream a slice of the partition's
// K and V tiles through a register ring and combine their states in LDS.
//   * Lane mapping: a wave reads one (block, head) tile [BS][D] as NL
//     coalesced 1 KiB loads: lane l takes 16 bytes of token row l / LPT at
//     dims (l % LPT) * E ... + E, where E = 16 / sizeof(elem) and
//     LPT = D / E lanes cover one row.
//   * QK^T: on the matrix cores for bf16 and 1-byte pools (below); for fp32
//     pools each lane multiplies its E key elements with the matching E
//     elements of the G (pre-scaled) queries held in registers, then a DPP
//     sum over the LPT lanes of the row gives the G scores.
//   * Scores go to LDS; the max and the sum of exp2(s - max) are taken over
//     the scores in LDS before PV (two-pass softmax inside the partition: no
//     running rescale of the accumulators).
//   * PV: bf16 and 1-byte pools on the matrix cores, V tiles staged in LDS
//     and read transposed (below); fp32 pools on the VALU with the same lane
//     mapping as the loads (each lane accumulates p[g][token] * v for its E
//     dims, then lanes of different rows are summed by shuffles).  The waves
//     of a partition combine their states through LDS.
//   * int8 pools (G <= 4) keep both products on the integer matrix cores:
//     q and the PV weights are split into four int8 limbs (fixed point
//     against the head's maximum, ~31 bits), the stored bytes enter
//     v_mfma_i32_16x16x64_i8 / _16x16x32_i8 unconverted and the int32 sums
//     are exact; fp8 pools convert their bytes to bf16 (exact).
// Pass 2 (decode_merge_kernel): per (query head, sequence) merge of the
// partition partials m (max), l (sum), acc (unnormalised PV):
//   M = max m_p;  out = sum_p 2^(m_p - M) acc_p / sum_p 2^(m_p - M) l_p.
// Sequences that fit one partition are finished in pass 1.
//
// Scores are kept in the log2 domain: the dot product is multiplied by
// scale * log2(e) (scale after the dot, as the reference applies it), so the
// softmax uses exp2 (v_exp_f32) directly.
#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>
#include <type_traits>

namespace rkv {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
// Upper bound on partitions per sequence the merge pass accepts (LDS weights):
// 2.6M tokens at 640 tokens per partition.
constexpr int kMaxMergeParts = 4096;  // 16 KiB of merge weights in LDS

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
template <>
struct Traits<uint8_t> {  // int8 / fp8 pools
  static constexpr int E = 16;
};

// Calls f(std::integral_constant<int, I>) for I = B .. E-1 in order.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Matrix-core operand types (bf16 and int8 MFMAs).
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) int i32x4_t;
typedef __attribute__((ext_vector_type(4))) short bf16x4_t;

// Converts one 16-byte load of an fp32 pool into 4 floats (16-bit pools
// reach the matrix cores as they are stored).
__device__ __forceinline__ void to_float(const uint4& w, float (&f)[4]) {
  f[0] = __uint_as_float(w.x);
  f[1] = __uint_as_float(w.y);
  f[2] = __uint_as_float(w.z);
  f[3] = __uint_as_float(w.w);
}

// The 4 stored bytes of a dword of a 1-byte pool as floats (before the row
// scale).  fp8: v_cvt_pk_f32_fp8, which decodes OCP e4m3 on gfx950 (checked
// against the exact bit decode for all 256 codes); int8: sign-extend + convert.
template <int FMT>
__device__ __forceinline__ void dword_values(uint32_t w, float (&f)[4]) {
  if constexpr (FMT == RKV_I8) {
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = (float)((int32_t)(w << (24 - 8 * e)) >> 24);
  } else {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);  // bytes 0, 1
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);   // bytes 2, 3
    f[0] = lo[0], f[1] = lo[1], f[2] = hi[0], f[3] = hi[1];
  }
}

// 16 stored bytes as floats (before the row scale).
template <int FMT>
__device__ __forceinline__ void to_float_q(const uint4& w, float (&f)[16]) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float t[4];
    dword_values<FMT>(ws[k], t);
#pragma unroll
    for (int e = 0; e < 4; ++e) f[4 * k + e] = t[e];
  }
}

// 8 stored bytes (two dwords) as 8 bf16 values packed in a uint4; exact, since
// int8 integers and e4m3 values have at most 8 significant bits.
template <int FMT>
__device__ __forceinline__ uint4 to_bf16x8_q(uint32_t lo, uint32_t hi) {
  if constexpr (FMT == RKV_FP8) {
    // v_cvt_scalef32_pk_bf16_fp8 with scale 1.0: two e4m3 bytes to two bf16
    // in one instruction (equal to the exact decode for all 256 codes, NaN
    // to NaN, checked on gfx950)
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
    const bf16x2_t a0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)lo, 1.0f, false);
    const bf16x2_t a1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)lo, 1.0f, true);
    const bf16x2_t b0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)hi, 1.0f, false);
    const bf16x2_t b1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)hi, 1.0f, true);
    return make_uint4(__builtin_bit_cast(uint32_t, a0), __builtin_bit_cast(uint32_t, a1),
                      __builtin_bit_cast(uint32_t, b0), __builtin_bit_cast(uint32_t, b1));
  }
  // int8: sign-extending byte converts, then one v_cvt_pk_bf16_f32 per pair
  // (exact: |value| <= 128)
  float a[4], b[4];
  dword_values<FMT>(lo, a);
  dword_values<FMT>(hi, b);
  return make_uint4(cvt_bf16x2(a[0], a[1]), cvt_bf16x2(a[2], a[3]), cvt_bf16x2(b[0], b[1]),
                    cvt_bf16x2(b[2], b[3]));
}

// The value of lane l + G within its 16-lane row, for the lanes l % 16 < G
// (other lanes receive another lane's value or 0): the lo-row column that
// pairs with hi column l of the MFMA PV result.  DPP inside the row:
// quad_perm xor 1 / xor 2, row_ror:8 (= xor 8); for G = 4 the sum of a
// row_shl:4 and a row_shr:4 move, one of which reads lane l + 4 while the
// other reads past the row edge and contributes 0.
template <int G>
__device__ __forceinline__ float lo_col(float x) {
  if constexpr (G == 4) return dpp<0x104>(x) + dpp<0x114>(x);
  constexpr int CTRL = G == 1 ? 0xB1 : G == 2 ? 0x4E : 0x128;
  return dpp<CTRL>(x);
}

// ---- streaming variant ---------------------------------------------------------
// SPLIT 64-lane waves own one (partition, KV head, sequence) item; a
// partition is SPLIT * tw blocks (tw = tiles_per_wave <= NTW = NTILE / SPLIT,
// chosen at launch), and wave w streams the tw tiles of its slice (the
// static loop runs over NTW slots; slots past tw are masked) -- the K
// tiles, then the V tiles -- through a ring of R register tiles: the loads of
// tile t + R are issued as soon as tile t has been consumed, so a wave always
// has R tiles (R KiB x 4 for bf16 D=128) in flight and its arithmetic overlaps
// its own loads.  Scores live in wave-private LDS; the only barrier is the
// final combine of the SPLIT softmax states (m, l, acc) through LDS.
// For bf16 pools QK^T runs on the matrix cores (MFMA = true): one
// v_mfma_f32_16x16x32_bf16 per 32 dims of a 16-token tile with
//   A (16 x 32) = queries: rows 0..G-1 = bf16(q) of the G heads, rows
//                 G..2G-1 = bf16(q - bf16(q)), other rows zero.  hi + lo keeps
//                 ~16 significant bits of q: scores as accurate as fp32 dots.
//   B (32 x 16) = K^T of the tile: lane l holds 16 bytes of token row l % 16
//                 at dims 32c + 8 (l / 16) (bf16).  K tiles are loaded like
//                 V tiles (contiguous token rows, 1 KiB per wave-load) and
//                 reach this layout through the wave's LDS staging buffer:
//                 loading it straight from the pool touches 16 rows x 64
//                 bytes per wave-load, half of every 128-byte line, which
//                 streams ~9% slower (RKV_DECODE_K_LDS=0 builds that form).
//   D (16 x 16) = row 4 (l / 16) + r in lane l register r, column l % 16.
// (Lane layout checked on gfx950: A[l%16][8(l/16)+e], B[8(l/16)+e][l%16],
// D[4(l/16)+r][l%16].)  PV runs on the matrix cores too (below); fp32 pools
// keep QK^T and PV on the VALU.
// Waves per SIMD the register allocation aims for: 3 keeps the bf16 and
// 1-byte kernels at D = 128, G <= 4 at 3 waves per SIMD without spilling.
#ifndef RKV_DECODE_WAVES_PER_SIMD
#define RKV_DECODE_WAVES_PER_SIMD 3
#endif
// bf16 K tiles through LDS (1) or loaded in the MFMA operand layout (0).
#ifndef RKV_DECODE_K_LDS
#define RKV_DECODE_K_LDS 1
#endif
// int8 pools: QK^T on v_mfma_i32_16x16x64_i8 with q in four int8 limbs (1)
// or on the bf16 MFMA with the K bytes converted (0); PV on
// v_mfma_i32_16x16x32_i8 with the weights in four int8 limbs (1) or on the
// bf16 MFMA with the V bytes converted (0).
#ifndef RKV_DECODE_I8_QK
#define RKV_DECODE_I8_QK 1
#endif
#ifndef RKV_DECODE_I8_PV
#define RKV_DECODE_I8_PV 1
#endif
// APPEND (bf16 pools): the step's new K/V rows (k_new / v_new, fp32
// [num_seqs][Hkv][D]) belong at position ctx_lens[b] - 1.  The wave whose
// slice holds that position stores them (bf16, rounded to nearest even as
// rkv_append does) into the pools before it streams its tiles, and reads
// them back with the rest of the tile.  Nothing else in the launch reads
// the row.
template <typename T, int D, int G, int BS, int NTILE, int R, int SPLIT, int FMT,
          bool APPEND = false>
__global__ __launch_bounds__(64 * SPLIT)
__attribute__((amdgpu_waves_per_eu(G >= 8 ? 2 : RKV_DECODE_WAVES_PER_SIMD))) void decode_stream_kernel(
    float* __restrict__ out, float* __restrict__ part_acc, float* __restrict__ part_ml,
    const float* __restrict__ q, const void* __restrict__ k_pool_,
    const void* __restrict__ v_pool_, const float* __restrict__ k_scale,
    const float* __restrict__ v_scale, const int32_t* __restrict__ block_tables,
    int max_blocks_per_seq, const int32_t* __restrict__ ctx_lens, int ctx_cap, int num_kv_heads,
    int64_t num_blocks, float q_scale, int max_parts, int tiles_per_wave,
    const float* __restrict__ k_new, const float* __restrict__ v_new) {
  const T* __restrict__ k_pool = static_cast<const T*>(k_pool_);
  const T* __restrict__ v_pool = static_cast<const T*>(v_pool_);
  constexpr int E = Traits<T>::E;
  constexpr int LPT = D / E;     // lanes per token row
  constexpr int TPL = 64 / LPT;  // token rows per wave-load
  constexpr int NL = BS / TPL;   // wave-loads per tile
  constexpr int NTW = NTILE / SPLIT;  // tile slots of this wave's slice
  const int tw = tiles_per_wave;      // tiles of the slice (1 .. NTW)
  const int P = tw * SPLIT * BS;      // tokens per partition
  constexpr int NT = 2 * NTW;    // tiles streamed: K then V
  static_assert(D % E == 0 && 64 % LPT == 0 && BS % TPL == 0 && R >= 1 && R <= NT,
                "unsupported tile shape");
  static_assert(NTILE % SPLIT == 0, "the partition splits evenly over the waves");

  // Per wave: scores, then probabilities; at the end the wave's (unnormalised)
  // output rows for the combine of the SPLIT slices (the same buffer: a wave
  // reads its probabilities before it writes its rows, and the combine reads
  // the rows only after the barrier).  One buffer instead of two keeps the
  // workgroup's LDS small enough for four workgroups per CU.
  constexpr int SPW = NTW * BS * G > G * D ? NTW * BS * G : G * D;
  __shared__ __align__(16) float s_pw[SPLIT][SPW];

  // The SPLIT waves stream consecutive NTW-tile slices of one partition and
  // combine their softmax states in LDS at the end.  The grid is KV-head
  // major: the Hkv workgroups of one (partition, sequence) are consecutive.
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kh = blockIdx.x, part = blockIdx.y, b = blockIdx.z;
  const int sub = w;
  float* __restrict__ s_p = s_pw[w];
  const int num_q_heads = num_kv_heads * G;
  const int lane = threadIdx.x & 63;
  const int slot = lane / LPT, dl = lane % LPT;
  const int64_t head0 = (int64_t)b * num_q_heads + kh * G;

  // Requests that do not depend on the context length go out first.
  int L = ctx_lens[b];
  const int L_raw = L;
  const int lb0 = (part * SPLIT + sub) * tw;  // first tile (block index) of this wave
  const int32_t* tab = block_tables + (int64_t)b * max_blocks_per_seq;
  int32_t pb[NTW];
#pragma unroll
  for (int i = 0; i < NTW; ++i) {
    const int lb = lb0 + i;
    const int lbc = lb < max_blocks_per_seq ? lb : max_blocks_per_seq - 1;
    pb[i] = lbc >= 0 ? tab[lbc] : -1;
  }
  // 1-byte pools (QNT): bytes plus one fp32 scale per (token, KV head) row.
  constexpr bool QNT = FMT == RKV_I8 || FMT == RKV_FP8;
  static_assert(QNT == (sizeof(T) == 1), "1-byte element type iff a 1-byte format");
  constexpr bool MFMA = (sizeof(T) == 2 || QNT) && 2 * G <= 16;
  // PV on the matrix cores as well (bf16 and 1-byte pools):
  // O^T[dim][col] += V^T[dim][key] P^T[key][col], A = V^T read with a
  // transposing LDS read from V tiles staged row-major in this wave's LDS
  // buffer, B = P^T with columns 0..G-1 = bf16(p) of the G heads and
  // G..2G-1 = bf16(p - bf16(p)) (1-byte pools: the V scale already folded
  // into p).  1-byte pools: a pair of tiles (32 keys) per
  // v_mfma_f32_16x16x32_bf16, ds_read_b64_tr_b8 (8 keys of one dim per lane),
  // converted to bf16 exactly.  bf16: one tile (16 keys) per
  // v_mfma_f32_16x16x16_bf16, ds_read_b64_tr_b16 (4 keys of one dim per lane),
  // which keeps the staging buffer at one tile.
  constexpr bool MPV = MFMA;
  // int8 pools (G <= 4): QK^T on the integer matrix cores, exact in int32.
  // q of head h is written as (M_h / 127) (a0 + a1 / 254 + a2 / 254^2 +
  // a3 / 254^3) with M_h = max |q| over the head's dims and int8 limbs a0 ..
  // a3 (round to nearest at each step; with the fp32 roundings of
  // q * 127 / M_h and of the residuals, |q - that sum| < |q| 2^-23 +
  // M_h 2^-31, where three limbs left M_h 2^-22: a component far under the
  // head's maximum keeps its own precision), the limbs are rows 4 h + j of
  // A, and B is the stored K bytes as they are.  Row 4 h + j of the result
  // lands in lane 16 h + token, register j: each lane combines the four
  // limb dots of one (head, token) pair in its own registers.  No
  // K byte is converted, and a 64-dim K block is one MFMA instead of two.
  constexpr bool I8QK = MFMA && FMT == RKV_I8 && G <= 4 && RKV_DECODE_I8_QK;
  // PV likewise: the weights w = p * (V row scale) of head h over the
  // wave's slice are written as (W_h / 127) (b0 + ... + b3 / 254^3) with
  // W_h = their maximum (so a row whose scale dwarfs the slice's others
  // leaves theirs ~2^-31 W_h of precision, not 2^-22), the limbs are the A rows 4 h + j (bytes in
  // LDS, written once per slice by the softmax pass), B is the staged V
  // bytes read transposed, and the int32 sums over the slice are exact.
  constexpr bool I8PV = MPV && FMT == RKV_I8 && G <= 4 && RKV_DECODE_I8_PV;
  constexpr int VROW = QNT ? D + 16 : 2 * (D + 16);  // staged V row (bytes): the rows of
                                                      // one transposing read hit distinct banks
  constexpr int NK = NTW * BS;   // keys of this wave's slice
  constexpr int VT = QNT ? 2 : 1;  // V tiles per staged group
  static_assert(!MPV || NTW % VT == 0, "MFMA PV takes 1-byte V tiles in pairs");
  __shared__ __align__(16) uint8_t s_vq[MPV ? SPLIT : 1][MPV ? VT * BS * VROW : 16];
  __shared__ __align__(16) float s_pq[MPV ? SPLIT : 1][MPV ? G * NK : 4];  // p, head-major
  f32x4_t ov[MPV && !I8PV ? D / 16 : 1];
#pragma unroll
  for (int c = 0; c < (MPV && !I8PV ? D / 16 : 1); ++c) ov[c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  i32x4_t iov[I8PV ? D / 16 : 1];  // I8PV: lane (kq, kt) rows 4 kq + r, dim 16 c + kt
#pragma unroll
  for (int c = 0; c < (I8PV ? D / 16 : 1); ++c) iov[c] = i32x4_t{0, 0, 0, 0};
  float pmul = 0.0f;  // I8PV: W_h / 127 of head kq (inf when a weight is NaN or inf)
  constexpr int NC = D / 32;                     // MFMAs per tile
  const int kt = lane & 15, kq = lane >> 4;      // MFMA lanes: token row, k-quarter
  // VALU path: this lane's E dims of each head.  MFMA path: the A operand
  // row kt (hi rows 0..G-1, lo rows G..2G-1), chunk c at dims 32c + 8 kq .. + 8
  // for bf16; for 1-byte pools a lane reads the contiguous quarter
  // [D/4 kq, D/4 (kq+1)) of its key row, so chunk c holds dims D/4 kq + 8c ..
  // + 8 (any assignment of dims to k-slots gives the same dot product, as long
  // as q and K use the same one).
  // I8QK: lane l loads dims (D/16) (l % 16) .. + D/16 of head l / 16 (the
  // limbs are built once per (head, dim) and exchanged through LDS).
  constexpr int QN = I8QK ? D / 16 : (MFMA ? NC * 8 : G * E);
  float qv[QN];
  if constexpr (I8QK) {
    const int hq = (lane >> 4) < G ? (lane >> 4) : 0;
#pragma unroll
    for (int e = 0; e < QN; e += 4) {
      const float4 x =
          *reinterpret_cast<const float4*>(q + (head0 + hq) * D + (lane & 15) * QN + e);
      qv[e + 0] = x.x; qv[e + 1] = x.y; qv[e + 2] = x.z; qv[e + 3] = x.w;
    }
  } else if constexpr (MFMA) {
    const int qrow = kt < G ? kt : (kt < 2 * G ? kt - G : 0);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d0 = QNT ? (D / 4) * kq + 8 * c : 32 * c + 8 * kq;
      const float4* qp = reinterpret_cast<const float4*>(q + (head0 + qrow) * D + d0);
      const float4 x = qp[0], y = qp[1];
      qv[c * 8 + 0] = x.x; qv[c * 8 + 1] = x.y; qv[c * 8 + 2] = x.z; qv[c * 8 + 3] = x.w;
      qv[c * 8 + 4] = y.x; qv[c * 8 + 5] = y.y; qv[c * 8 + 6] = y.z; qv[c * 8 + 7] = y.w;
    }
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float* qp = q + (head0 + g) * D + dl * E;
#pragma unroll
      for (int e = 0; e < E; e += 4) {
        const float4 v = *reinterpret_cast<const float4*>(qp + e);
        qv[g * E + e + 0] = v.x;
        qv[g * E + e + 1] = v.y;
        qv[g * E + e + 2] = v.z;
        qv[g * E + e + 3] = v.w;
      }
    }
  }



  L = L < 0 ? 0 : (L > ctx_cap ? ctx_cap : L);
  const int nparts = (L + P - 1) / P;
  if (L == 0) {
    if (part == 0 && sub == 0)
      for (int o = lane; o < G * D; o += 64) out[head0 * D + o] = 0.0f;
    return;
  }
  if (part >= nparts) return;

  // Tile i of the partition is block lb0 + i.  A tile past the context, or
  // with an invalid id, re-reads tile 0 (an L2 hit) and is masked.  Block ids
  // are int32, so validity is one unsigned compare against the pool size
  // clamped to 2^31 - 1.
  const uint32_t nb32 = num_blocks > 0x7fffffff ? 0x7fffffffu : (uint32_t)num_blocks;
  const int32_t pb0 = (uint32_t)pb[0] < nb32 ? pb[0] : 0;
  int64_t base[NTW];  // wave-uniform element offset of each (block, head) tile
  bool ok[NTW], full[NTW];
#pragma unroll
  for (int i = 0; i < NTW; ++i) {
    const int tbase = (lb0 + i) * BS;
    ok[i] = i < tw && tbase < L && (uint32_t)pb[i] < nb32;
    full[i] = ok[i] && tbase + BS <= L;
    base[i] = ((int64_t)(ok[i] ? pb[i] : pb0) * num_kv_heads + kh) * BS * D;
  }
  // This lane's byte offset in a (block, head) tile and the stride between
  // its loads.  A masked tile re-reads the wave's tile 0 (its streaming
  // re-reads add ~2% to FETCH_SIZE; masking them with an empty buffer
  // resource instead removed that traffic but made the kernel ~4% slower).
  // MFMA: K tiles staged through LDS are loaded like V tiles.
  constexpr bool KLDS = MFMA && RKV_DECODE_K_LDS;
  constexpr int KROW = D * sizeof(T) + 16;  // staged K row (bytes): the 16 rows
                                            // of one operand read hit distinct banks
  static_assert(!KLDS || BS * KROW <= VT * BS * VROW, "K staging fits the V staging buffer");
  static_assert(!I8QK || BS * KROW + 16 * D <= VT * BS * VROW,
                "K staging and the q limb rows fit the V staging buffer");
  constexpr bool kmfma = MFMA && !KLDS;
  const uint32_t koff = (kmfma ? kt * D + (QNT ? (D / 4) * kq : 8 * kq) : slot * D + dl * E) * sizeof(T);
  const uint32_t voff = (slot * D + dl * E) * sizeof(T);
  constexpr uint32_t KSTEP = (kmfma ? (QNT ? 16 : 32) : TPL * D) * sizeof(T);
  constexpr uint32_t VSTEP = TPL * D * sizeof(T);
  auto tile_load = [&](int t, int n) __attribute__((always_inline)) {
    const bool is_k = t < NTW;
    const int i = t % NTW;
    return load_stream(reinterpret_cast<const char*>((is_k ? k_pool : v_pool) + base[i]) +
                       (is_k ? koff : voff) + n * (is_k ? KSTEP : VSTEP));
  };

  // APPEND: the wave whose slice holds position L - 1 stores the new K and V
  // rows (bf16) into the pools before its ring loads and waits for the
  // stores; the lanes that store a row piece are the lanes whose ring load
  // reads it back (row n TPL + slot, piece dl), so the loop sees the new row
  // with no other change.  The stores wait only in this one wave of the
  // sequence's last partition.  A block id outside the pool (rkv_append
  // skips those slots) or a length clamped to ctx_cap stores nothing.
  static_assert(!APPEND || sizeof(T) == 2 || QNT, "the fused append: bf16 and 1-byte pools");
  if constexpr (APPEND && QNT) {
    // 1-byte pools: rkv_append_q's quantization of the row (maximum |x| of
    // the row over its LPT lanes, bytes of x * top / max, scale max / top)
    const int tn = L - 1, ti = tn / BS;
    if (L_raw == L && ti >= lb0 && ti < lb0 + tw) {  // wave-uniform
      const int r = tn - ti * BS;
      const int32_t blk = tab[ti];
      if ((uint32_t)blk < nb32 && slot == r % TPL) {  // whole LPT-lane groups
        constexpr float kTop = FMT == RKV_I8 ? 127.0f : 448.0f;
        const int64_t src = ((int64_t)b * num_kv_heads + kh) * D + dl * E;
        const int64_t row = ((int64_t)blk * num_kv_heads + kh) * BS + r;
        float kx[E], vx[E];
#pragma unroll
        for (int e = 0; e < E; e += 4) {
          const float4 k4 = *reinterpret_cast<const float4*>(k_new + src + e);
          const float4 v4 = *reinterpret_cast<const float4*>(v_new + src + e);
          kx[e] = k4.x, kx[e + 1] = k4.y, kx[e + 2] = k4.z, kx[e + 3] = k4.w;
          vx[e] = v4.x, vx[e + 1] = v4.y, vx[e + 2] = v4.z, vx[e + 3] = v4.w;
        }
        float ka = 0.0f, va = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          ka = fmaxf(ka, fabsf(kx[e]));
          va = fmaxf(va, fabsf(vx[e]));
        }
        ka = group_max<LPT>(ka);
        va = group_max<LPT>(va);
        const float kinv = ka > 0.0f ? kTop / ka : 0.0f, vinv = va > 0.0f ? kTop / va : 0.0f;
        uint32_t kw[4] = {0u, 0u, 0u, 0u}, vw[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const uint32_t kb = FMT == RKV_I8 ? i8_quant(kx[e], kinv) : e4m3_from_f32(kx[e] * kinv);
          const uint32_t vb = FMT == RKV_I8 ? i8_quant(vx[e], vinv) : e4m3_from_f32(vx[e] * vinv);
          kw[e >> 2] |= kb << (8 * (e & 3));
          vw[e >> 2] |= vb << (8 * (e & 3));
        }
        *reinterpret_cast<uint4*>(const_cast<T*>(k_pool) + row * D + dl * E) =
            make_uint4(kw[0], kw[1], kw[2], kw[3]);
        *reinterpret_cast<uint4*>(const_cast<T*>(v_pool) + row * D + dl * E) =
            make_uint4(vw[0], vw[1], vw[2], vw[3]);
        if (dl == 0) {
          const_cast<float*>(k_scale)[row] = ka / kTop;
          const_cast<float*>(v_scale)[row] = va / kTop;
        }
      }
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the stores are done in L2
    }
  } else if constexpr (APPEND) {
    const int tn = L - 1, ti = tn / BS;
    if (L_raw == L && ti >= lb0 && ti < lb0 + tw) {  // wave-uniform
      const int r = tn - ti * BS;
      const int32_t blk = tab[ti];
      if ((uint32_t)blk < nb32 && slot == r % TPL) {
        const int64_t src = ((int64_t)b * num_kv_heads + kh) * D + dl * E;
        const int64_t dst = (((int64_t)blk * num_kv_heads + kh) * BS + r) * D + dl * E;
        const float4 k0 = *reinterpret_cast<const float4*>(k_new + src);
        const float4 k1 = *reinterpret_cast<const float4*>(k_new + src + 4);
        const float4 v0 = *reinterpret_cast<const float4*>(v_new + src);
        const float4 v1 = *reinterpret_cast<const float4*>(v_new + src + 4);
        *reinterpret_cast<uint4*>(const_cast<T*>(k_pool) + dst) =
            make_uint4(pack_bf16x2(k0.x, k0.y), pack_bf16x2(k0.z, k0.w),
                       pack_bf16x2(k1.x, k1.y), pack_bf16x2(k1.z, k1.w));
        *reinterpret_cast<uint4*>(const_cast<T*>(v_pool) + dst) =
            make_uint4(pack_bf16x2(v0.x, v0.y), pack_bf16x2(v0.z, v0.w),
                       pack_bf16x2(v1.x, v1.y), pack_bf16x2(v1.z, v1.w));
      }
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the stores are done in L2
    }
  }

  const int tok0 = lb0 * BS;  // first token of this wave's slice
  float acc[G][E];
  float m[G], l[G];
  uint4 ring[R][NL];
#pragma unroll
  for (int t = 0; t < R; ++t) {
#pragma unroll
    for (int n = 0; n < NL; ++n) ring[t][n] = tile_load(t, n);
  }

  // 1-byte pools: the K scale of this lane's token in each K tile (MFMA column
  // kt), and the V scale of the tokens this lane folds into the
  // probabilities (x = lane + 64 j of the slice).  Issued with the ring loads.
  // APPEND: a scale the wave stored is read by other lanes, and a 128-byte
  // line of scales spans two KV heads' tiles, which another workgroup on the
  // CU may have cached in L1: these loads read L2.
  constexpr int NX = QNT ? (NTW * BS + 63) / 64 : 1;
  float ksc[QNT ? NTW : 1], vsc[NX];
  auto ld_scale = [](const float* p) __attribute__((always_inline)) {
    if constexpr (APPEND) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *p;
  };
  if constexpr (QNT) {
#pragma unroll
    for (int i = 0; i < NTW; ++i) ksc[i] = ld_scale(k_scale + base[i] / D + kt);
#pragma unroll
    for (int j = 0; j < NX; ++j) {
      const int x = lane + 64 * j, ix = x / BS;
      int64_t rb = base[0];  // base[ix] by selects (ix differs between lanes)
#pragma unroll
      for (int i = 1; i < NTW; ++i) rb = ix == i ? base[i] : rb;
      vsc[j] = x < NTW * BS ? ld_scale(v_scale + rb / D + x % BS) : 0.0f;
    }
  }

  // q was requested before the ring and is converted after it: the barrier
  // keeps the conversion (which waits for q) below the ring's requests --
  // without it the scheduler interleaves the two and the first tile is not
  // requested until q has arrived.
  __builtin_amdgcn_sched_barrier(0);
  // MFMA A operands: q split into bf16 hi + lo rows, two values per
  // v_cvt_pk_bf16_f32 (round to nearest even, no branch)
  uint4 qa[MFMA ? NC : 1];
  float qmul = 0.0f;  // I8QK: M_h / 127 of head kq (inf when q_h holds NaN or inf)
  if constexpr (I8QK) {
    // M_h over the 16 lanes of head l / 16 (a NaN counts as inf: the limbs
    // are then zero and the head's dots 0 * inf = NaN, as in the float path)
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < QN; ++e) amax = fmaxf(amax, qv[e] != qv[e] ? INFINITY : fabsf(qv[e]));
    amax = group_max<16>(amax);
    const float inv = amax >= 0x1p-120f ? 127.0f / amax : 0.0f;  // finite
    // limb rows 4 h + j of D bytes each, after the K staging rows
    uint8_t* qbuf = s_vq[w] + BS * KROW;
    uint32_t lw[4][QN / 4];
#pragma unroll
    for (int e4 = 0; e4 < QN / 4; ++e4) {
      lw[0][e4] = lw[1][e4] = lw[2][e4] = lw[3][e4] = 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = qv[4 * e4 + e] * inv;  // |a| <= 127
        const float a0 = rintf(a);
        const float r1 = (a - a0) * 254.0f;  // |r1| <= 127
        const float a1 = rintf(r1);
        const float r2 = (r1 - a1) * 254.0f;
        const float a2 = rintf(r2);
        const float a3 = rintf((r2 - a2) * 254.0f);
        lw[0][e4] |= ((uint32_t)(int32_t)a0 & 0xffu) << (8 * e);
        lw[1][e4] |= ((uint32_t)(int32_t)a1 & 0xffu) << (8 * e);
        lw[2][e4] |= ((uint32_t)(int32_t)a2 & 0xffu) << (8 * e);
        lw[3][e4] |= ((uint32_t)(int32_t)a3 & 0xffu) << (8 * e);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint8_t* dst = qbuf + (4 * (lane >> 4) + j) * D + (lane & 15) * QN;
      if constexpr (QN == 8)
        *reinterpret_cast<uint2*>(dst) = make_uint2(lw[j][0], lw[j][1]);
      else
        *reinterpret_cast<uint32_t*>(dst) = lw[j][0];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the limb rows ...
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");  // ... before the reads
    // A row kt: head kt / 4, limb kt % 4 (heads >= G are zero rows)
    const bool live = kt / 4 < G;
#pragma unroll
    for (int n = 0; n < NL; ++n) {
      const uint4 v = *reinterpret_cast<const uint4*>(
          qbuf + (live ? kt : 0) * D + (D / 4) * kq + 16 * n);
      qa[n] = live ? v : make_uint4(0u, 0u, 0u, 0u);
    }
    // this lane's result rows belong to head kq, whose M_h this lane holds
    qmul = amax * (1.0f / 127.0f);
  } else if constexpr (MFMA) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      uint32_t h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = qv[c * 8 + 2 * e], y = qv[c * 8 + 2 * e + 1];
        const uint32_t hi = cvt_bf16x2(x, y);
        const uint32_t lo =
            cvt_bf16x2(x - __uint_as_float(hi << 16), y - __uint_as_float(hi & 0xffff0000u));
        h[e] = kt < G ? hi : (kt < 2 * G ? lo : 0u);
      }
      qa[c] = make_uint4(h[0], h[1], h[2], h[3]);
    }
  }

  // The 2*NTW steps are instantiated one by one (static_for) so that every
  // ring slot is a fixed set of registers.
  static_for<0, NT>([&](auto tc) __attribute__((always_inline)) {
    constexpr int t = decltype(tc)::value;
    constexpr int i = t % NTW;
    uint4* tile = ring[t % R];
    // Refill the slot just consumed with tile t + R; the refill's loads issue
    // at raised wave priority, ahead of the other waves' arithmetic on the
    // SIMD (about 1% at configs[2]).  A tile staged in LDS frees its slot
    // once written there, before the step's arithmetic.
    auto refill = [&]() __attribute__((always_inline)) {
      if constexpr (t + R < NT) {
        constexpr int tn = t + R;
        __builtin_amdgcn_s_setprio(3);
#pragma unroll
        for (int n = 0; n < NL; ++n) tile[n] = tile_load(tn, n);
        __builtin_amdgcn_s_setprio(0);
      }
    };
    constexpr bool staged = t < NTW ? KLDS : MPV;
    if constexpr (t < NTW) {
      // ---- QK^T for the 16 tokens of tile i ----
      if constexpr (MFMA) {
        f32x4_t sacc = {0.0f, 0.0f, 0.0f, 0.0f};
        // This lane's K operand: NL 16-byte pieces of token kt (bf16: dims
        // 32c + 8 kq .. + 7 for MFMA c; 1-byte: bytes (D/4) kq + 16 n .. + 15).
        uint4 kb[NL];
        if constexpr (KLDS) {
          // rows to LDS (token n TPL + slot, 16 bytes at element E dl), the
          // ring slot refilled, then the operand pieces read back
          uint8_t* kbuf = s_vq[w];
#pragma unroll
          for (int n = 0; n < NL; ++n)
            *reinterpret_cast<uint4*>(kbuf + (n * TPL + slot) * KROW + dl * 16) = tile[n];
          if constexpr (staged) refill();
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the rows ...
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");  // ... before the reads
#pragma unroll
          for (int n = 0; n < NL; ++n)
            kb[n] = *reinterpret_cast<const uint4*>(
                kbuf + kt * KROW + (QNT ? (D / 4) * kq + 16 * n : 64 * n + 16 * kq));
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // reads done before
          __builtin_amdgcn_wave_barrier();                         // the next tile's rows
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        } else {
#pragma unroll
          for (int n = 0; n < NL; ++n) kb[n] = tile[n];
        }
        if constexpr (I8QK) {
          i32x4_t iacc = {0, 0, 0, 0};
#pragma unroll
          for (int n = 0; n < NL; ++n)
            iacc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4_t, qa[n]),
                                                         __builtin_bit_cast(i32x4_t, kb[n]),
                                                         iacc, 0, 0, 0);
          sacc[0] = ((float)iacc[0] + (float)iacc[1] * (1.0f / 254.0f) +
                     (float)iacc[2] * (1.0f / 64516.0f) +
                     (float)iacc[3] * (1.0f / 16387064.0f)) * qmul;
        } else if constexpr (QNT) {
#pragma unroll
          for (int n = 0; n < NL; ++n) {
            sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8_t, qa[2 * n]),
                __builtin_bit_cast(bf16x8_t, to_bf16x8_q<FMT>(kb[n].x, kb[n].y)), sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8_t, qa[2 * n + 1]),
                __builtin_bit_cast(bf16x8_t, to_bf16x8_q<FMT>(kb[n].z, kb[n].w)), sacc, 0, 0, 0);
          }
        } else {
          static_assert(QNT || NL == NC, "one 16-byte K piece per MFMA");
#pragma unroll
          for (int c = 0; c < NC; ++c)
            sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, qa[c]),
                                                          __builtin_bit_cast(bf16x8_t, kb[c]),
                                                          sacc, 0, 0, 0);
        }
        // dot * scale (the reference's order), then the token's K row scale
        float qs = q_scale;
        if constexpr (QNT) qs *= ksc[i];
        const int tp = i * BS + kt;  // token of this lane's column
        const bool valid = ok[i] && (tok0 + tp < L);
        if constexpr (I8QK) {
          if (kq < G) s_p[tp * G + kq] = valid ? sacc[0] * qs : -INFINITY;
        } else if constexpr (G == 1) {
          if (kq == 0) s_p[tp] = valid ? (sacc[0] + sacc[1]) * qs : -INFINITY;
        } else if constexpr (G == 2) {
          if (kq == 0) {
            s_p[tp * 2 + 0] = valid ? (sacc[0] + sacc[2]) * qs : -INFINITY;
            s_p[tp * 2 + 1] = valid ? (sacc[1] + sacc[3]) * qs : -INFINITY;
          }
        } else {
          constexpr int XOR = G == 4 ? 16 : 32;  // lanes between hi and lo rows
          float sc[4];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            sc[r] = (XOR == 16 ? pair16_sum(sacc[r]) : pair32_sum(sacc[r])) * qs;
          if (lane < XOR) {  // lanes kq * 16 + kt hold heads 4 kq .. 4 kq + 3
            *reinterpret_cast<float4*>(&s_p[tp * G + 4 * kq]) =
                valid ? make_float4(sc[0], sc[1], sc[2], sc[3])
                      : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
          }
        }
      } else {
#pragma unroll
        for (int n = 0; n < NL; ++n) {
          float kf[E];
          to_float(tile[n], kf);
          float sc[G];
#pragma unroll
          for (int g = 0; g < G; ++g) {
            float a = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) a = fmaf(qv[g * E + e], kf[e], a);
            sc[g] = group_sum<LPT>(a) * q_scale;  // scale after the dot
          }
          const int tp = i * BS + n * TPL + slot;
          const bool valid = ok[i] && (tok0 + tp < L);
          if (dl == 0) {
#pragma unroll
            for (int g = 0; g < G; ++g) s_p[tp * G + g] = valid ? sc[g] : -INFINITY;
          }
        }
      }
      if constexpr (t == NTW - 1) {
        // ---- softmax statistics over the partition (this wave only) ----
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // LDS writes above ...
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");  // ... before the reads below
#pragma unroll
        for (int g = 0; g < G; ++g) m[g] = -INFINITY;
#pragma unroll
        for (int x = lane; x < NTW * BS; x += 64)
#pragma unroll
          for (int g = 0; g < G; ++g) m[g] = fmaxf(m[g], s_p[x * G + g]);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          m[g] = wave_max(m[g]);
          l[g] = 0.0f;
        }
        if constexpr (I8PV) {
          // weights in registers, their maximum per head, then the limbs
          constexpr int NJ = (NK + 63) / 64;
          float wv[NJ][G];
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const int x = lane + 64 * j;
#pragma unroll
            for (int g = 0; g < G; ++g) {
              const float sv = x < NK ? s_p[x * G + g] : -INFINITY;
              const float pv = (sv == -INFINITY) ? 0.0f : exp2f(sv - m[g]);
              l[g] += pv;
              wv[j][g] = pv > 0.0f ? pv * vsc[j] : 0.0f;  // masked: the scale never enters
            }
          }
          uint8_t* s_w8 = reinterpret_cast<uint8_t*>(s_pq[w]);  // rows 4 g + limb, NK bytes
#pragma unroll
          for (int g = 0; g < G; ++g) {
            // a NaN weight counts as inf: the limbs are then zero and the
            // head's sums 0 * inf = NaN, as in the float path
            float wm = 0.0f;
#pragma unroll
            for (int j = 0; j < NJ; ++j) wm = fmaxf(wm, wv[j][g] != wv[j][g] ? INFINITY : wv[j][g]);
            wm = wave_max(wm);
            const float inv = wm >= 0x1p-120f ? 127.0f / wm : 0.0f;
            pmul = kq == g ? wm * (1.0f / 127.0f) : pmul;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
              const int x = lane + 64 * j;
              if (x < NK) {
                const float a = wv[j][g] * inv;  // 0 <= a <= 127
                const float b0 = rintf(a);
                const float r1 = (a - b0) * 254.0f;
                const float b1 = rintf(r1);
                const float r2 = (r1 - b1) * 254.0f;
                const float b2 = rintf(r2);
                const float b3 = rintf((r2 - b2) * 254.0f);
                s_w8[(4 * g + 0) * NK + x] = (uint8_t)(int32_t)b0;
                s_w8[(4 * g + 1) * NK + x] = (uint8_t)(int32_t)b1;
                s_w8[(4 * g + 2) * NK + x] = (uint8_t)(int32_t)b2;
                s_w8[(4 * g + 3) * NK + x] = (uint8_t)(int32_t)b3;
              }
            }
          }
        } else {
#pragma unroll
        for (int j = 0; j < (NTW * BS + 63) / 64; ++j) {
          const int x = lane + 64 * j;
          if (x < NTW * BS) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
              const float sv = s_p[x * G + g];
              const float pv = (sv == -INFINITY) ? 0.0f : exp2f(sv - m[g]);
              l[g] += pv;
              // 1-byte pools: the V row scale goes into the weight (selected,
              // so the unwritten scale of a masked token never enters)
              if constexpr (MPV && QNT)
                s_pq[w][g * NK + x] = pv > 0.0f ? pv * vsc[j] : 0.0f;
              else if constexpr (MPV)
                s_pq[w][g * NK + x] = pv;
              else if constexpr (QNT)
                s_p[x * G + g] = pv > 0.0f ? pv * vsc[j] : 0.0f;
              else
                s_p[x * G + g] = pv;
            }
          }
        }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          l[g] = wave_sum(l[g]);
#pragma unroll
          for (int e = 0; e < E; ++e) acc[g][e] = 0.0f;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    } else if constexpr (MPV) {
      // ---- PV on the matrix cores ----
      // Stage tile i's rows into this wave's buffer (half i & 1 for 1-byte
      // pairs); rows past the context or of a bad block id are zeroed (a NaN
      // element times a zero p would still be NaN).
      const int tbase = (lb0 + i) * BS;
      uint8_t* vb = s_vq[w];
      if (full[i]) {  // wave-uniform: every row of the tile is valid, no selects
#pragma unroll
        for (int n = 0; n < NL; ++n)
          *reinterpret_cast<uint4*>(vb + ((i % VT) * BS + n * TPL + slot) * VROW + dl * 16) =
              tile[n];
      } else {
#pragma unroll
        for (int n = 0; n < NL; ++n) {
          const bool keep = ok[i] & (tbase + n * TPL + slot < L);
          uint4 vv = tile[n];
          vv.x = keep ? vv.x : 0u;
          vv.y = keep ? vv.y : 0u;
          vv.z = keep ? vv.z : 0u;
          vv.w = keep ? vv.w : 0u;
          *reinterpret_cast<uint4*>(vb + ((i % VT) * BS + n * TPL + slot) * VROW + dl * 16) = vv;
        }
      }
      if constexpr (staged) refill();
      if constexpr (!QNT) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the tile's rows ...
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");  // ... before the reads below
        // B = P^T (16 x 16 x 16): k-slot 4 kq + e holds key 4 kq + e of the
        // tile, column kt
        const int pc = kt < G ? kt : (kt < 2 * G ? kt - G : 0);
        const float4 p4 = *reinterpret_cast<const float4*>(&s_pq[w][pc * NK + i * BS + 4 * kq]);
        const uint32_t h0 = cvt_bf16x2(p4.x, p4.y), h1 = cvt_bf16x2(p4.z, p4.w);
        const uint32_t l0 =
            cvt_bf16x2(p4.x - __uint_as_float(h0 << 16), p4.y - __uint_as_float(h0 & 0xffff0000u));
        const uint32_t l1 =
            cvt_bf16x2(p4.z - __uint_as_float(h1 << 16), p4.w - __uint_as_float(h1 & 0xffff0000u));
        const uint2 pb = kt < G ? make_uint2(h0, h1)
                                : (kt < 2 * G ? make_uint2(l0, l1) : make_uint2(0u, 0u));
        // A = V^T: this lane's read address is key 4 kq + (kt >> 2), dims
        // 16 c + 4 (kt & 3) .. + 3
        const uint8_t* va = vb + (4 * kq + (kt >> 2)) * VROW + 8 * (kt & 3);
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
          const uint2 a = lds_read_tr16(va + 32 * c);
          ov[c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
              __builtin_bit_cast(bf16x4_t, a), __builtin_bit_cast(bf16x4_t, pb), ov[c], 0, 0, 0);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // reads done before the
        __builtin_amdgcn_wave_barrier();                         // next tile overwrites
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      } else if constexpr ((i & 1) && I8PV) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the pair's rows ...
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");  // ... before the reads below
        // A = weight limbs: lane (kq, kt) holds row kt (head kt / 4, limb
        // kt % 4; heads >= G are zero rows), keys 8 kq .. + 7 of the pair
        const uint8_t* s_w8 = reinterpret_cast<const uint8_t*>(s_pq[w]);
        const bool arow = kt < 4 * G;
        const uint2 wa = *reinterpret_cast<const uint2*>(
            s_w8 + (arow ? kt : 0) * NK + (i - 1) * BS + 8 * kq);
        const long pa = arow ? __builtin_bit_cast(long, wa) : 0l;
        // B = V: lane (kq, kt) holds keys 8 kq .. + 7 of dim 16 c + kt (the
        // transposing read of the bf16 path's A operand)
        const uint8_t* va = vb + (8 * kq + (kt >> 1)) * VROW + 8 * (kt & 1);
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
          const uint2 raw = lds_read_tr8(va + 16 * c);
          iov[c] = __builtin_amdgcn_mfma_i32_16x16x32_i8(pa, __builtin_bit_cast(long, raw),
                                                         iov[c], 0, 0, 0);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // reads done before the
        __builtin_amdgcn_wave_barrier();                         // next pair overwrites
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      } else if constexpr (i & 1) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the pair's rows ...
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");  // ... before the reads below
        // B = P^T: lane (kq, kt) holds keys 8 kq .. + 7 of the pair, column kt
        const int pc = kt < G ? kt : (kt < 2 * G ? kt - G : 0);
        const float* pp = &s_pq[w][pc * NK + (i - 1) * BS + 8 * kq];
        const float4 p0 = reinterpret_cast<const float4*>(pp)[0];
        const float4 p1 = reinterpret_cast<const float4*>(pp)[1];
        const float pv8[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
        uint32_t pw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = pv8[2 * e], y = pv8[2 * e + 1];
          const uint32_t hi = cvt_bf16x2(x, y);  // round to nearest even (p is finite)
          const uint32_t lo =
              cvt_bf16x2(x - __uint_as_float(hi << 16), y - __uint_as_float(hi & 0xffff0000u));
          pw[e] = kt < G ? hi : (kt < 2 * G ? lo : 0u);
        }
        const uint4 pb = make_uint4(pw[0], pw[1], pw[2], pw[3]);
        // A = V^T, 16 dims per MFMA: this lane's read address is key
        // 8 kq + (kt >> 1), bytes 16 c + 8 (kt & 1) .. + 7
        const uint8_t* va = vb + (8 * kq + (kt >> 1)) * VROW + 8 * (kt & 1);
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
          const uint2 raw = lds_read_tr8(va + 16 * c);
          ov[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, to_bf16x8_q<FMT>(raw.x, raw.y)),
              __builtin_bit_cast(bf16x8_t, pb), ov[c], 0, 0, 0);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // reads done before the
        __builtin_amdgcn_wave_barrier();                         // next pair overwrites
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    } else {
      // ---- PV for the 16 tokens of tile i ----
      // Rows past the context (or of a bad block id) are zeroed with selects,
      // not branches: branches here let the compiler sink every PV FMA to the
      // end of the kernel and keep all V tiles live.
      const int tbase = (lb0 + i) * BS;
#pragma unroll
      for (int n = 0; n < NL; ++n) {
        const bool keep = ok[i] & (tbase + n * TPL + slot < L);
        uint4 vv = tile[n];
        vv.x = keep ? vv.x : 0u;
        vv.y = keep ? vv.y : 0u;
        vv.z = keep ? vv.z : 0u;
        vv.w = keep ? vv.w : 0u;
        float vf[E];
        if constexpr (QNT)
          to_float_q<FMT>(vv, vf);
        else
          to_float(vv, vf);
        const int tp = i * BS + n * TPL + slot;
        float pr[G];
#pragma unroll
        for (int g = 0; g < G; ++g) pr[g] = s_p[tp * G + g];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int e = 0; e < E; ++e) acc[g][e] = fmaf(pr[g], vf[e], acc[g][e]);
      }
    }
    if constexpr (!staged) refill();
    // keep the ring a ring: the scheduler may not hoist later refills above
    // this step's arithmetic (that would need all 2*NTW tiles in registers)
    __builtin_amdgcn_sched_barrier(0);
  });

  // MFMA PV: lane (kq, kt) holds O^T[dim 16 c + 4 kq + r][column kt]; head
  // g's sum is column g (hi) plus column G + g (lo): lanes kt < G take it.
  // I8PV: lane (kq, kt) holds head kq's sums for dims 16 c + kt.
  f32x4_t hv[MPV && !I8PV ? D / 16 : 1];
  float iv[I8PV ? D / 16 : 1];
  if constexpr (I8PV) {
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
      iv[c] = ((float)iov[c][0] + (float)iov[c][1] * (1.0f / 254.0f) +
               (float)iov[c][2] * (1.0f / 64516.0f) +
               (float)iov[c][3] * (1.0f / 16387064.0f)) * pmul;
  } else if constexpr (MPV) {
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) hv[c][r] = ov[c][r] + lo_col<G>(ov[c][r]);
  } else {
    // sum over the TPL token rows, then lanes of row 0 hold the result
#pragma unroll
    for (int o = LPT; o < 64; o <<= 1)
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[g][e] += __shfl_xor(acc[g][e], o);
  }
  if constexpr (SPLIT == 1 && I8PV) {
    if (kq < G) {
      float mg = m[0], lg = l[0];  // head kq's state
#pragma unroll
      for (int x = 1; x < G; ++x) {
        mg = kq == x ? m[x] : mg;
        lg = kq == x ? l[x] : lg;
      }
      float* dst;
      float scl = 1.0f;
      if (nparts == 1) {
        dst = out + (head0 + kq) * D;
        scl = lg > 0.0f ? 1.0f / lg : 0.0f;
      } else {
        const int64_t row = (head0 + kq) * max_parts + part;
        dst = part_acc + row * D;
        if (kt == 0) {
          part_ml[row * 2 + 0] = mg;
          part_ml[row * 2 + 1] = lg;
        }
      }
#pragma unroll
      for (int c = 0; c < D / 16; ++c) dst[16 * c + kt] = iv[c] * scl;
    }
  } else if constexpr (SPLIT == 1 && MPV) {
    if (kt < G) {
      float mg = m[0], lg = l[0];  // head kt's state (selects: kt is not constant)
#pragma unroll
      for (int x = 1; x < G; ++x) {
        mg = kt == x ? m[x] : mg;
        lg = kt == x ? l[x] : lg;
      }
      float* dst;
      float scl = 1.0f;
      if (nparts == 1) {
        dst = out + (head0 + kt) * D;
        scl = lg > 0.0f ? 1.0f / lg : 0.0f;
      } else {
        const int64_t row = (head0 + kt) * max_parts + part;
        dst = part_acc + row * D;
        if (kq == 0) {
          part_ml[row * 2 + 0] = mg;
          part_ml[row * 2 + 1] = lg;
        }
      }
#pragma unroll
      for (int c = 0; c < D / 16; ++c)
        *reinterpret_cast<float4*>(dst + 16 * c + 4 * kq) =
            make_float4(hv[c][0] * scl, hv[c][1] * scl, hv[c][2] * scl, hv[c][3] * scl);
    }
  } else if constexpr (SPLIT == 1) {
    if (slot == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float* dst;
        float scl = 1.0f;
        if (nparts == 1) {
          dst = out + (head0 + g) * D + dl * E;
          scl = l[g] > 0.0f ? 1.0f / l[g] : 0.0f;
        } else {
          const int64_t row = (head0 + g) * max_parts + part;
          dst = part_acc + row * D + dl * E;
          if (dl == 0) {
            part_ml[row * 2 + 0] = m[g];
            part_ml[row * 2 + 1] = l[g];
          }
        }
#pragma unroll
        for (int e = 0; e < E; e += 4)
          *reinterpret_cast<float4*>(dst + e) =
              make_float4(acc[g][e] * scl, acc[g][e + 1] * scl, acc[g][e + 2] * scl,
                          acc[g][e + 3] * scl);
      }
    }
  } else {
    // Combine the SPLIT slices: M = max m_s, w_s = 2^(m_s - M),
    // l = sum w_s l_s, acc = sum w_s acc_s (a slice without a valid token has
    // m = -inf and weight 0).
    __shared__ float s_cm[SPLIT][G], s_cl[SPLIT][G];
    float(*s_cacc)[SPW] = s_pw;
    if constexpr (I8PV) {
      if (kq < G) {
#pragma unroll
        for (int c = 0; c < D / 16; ++c) s_cacc[sub][kq * D + 16 * c + kt] = iv[c];
      }
      if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          s_cm[sub][g] = m[g];
          s_cl[sub][g] = l[g];
        }
      }
    } else if constexpr (MPV) {
      if (kt < G) {
#pragma unroll
        for (int c = 0; c < D / 16; ++c)
          *reinterpret_cast<float4*>(&s_cacc[sub][kt * D + 16 * c + 4 * kq]) =
              make_float4(hv[c][0], hv[c][1], hv[c][2], hv[c][3]);
      }
      if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          s_cm[sub][g] = m[g];
          s_cl[sub][g] = l[g];
        }
      }
    } else if (slot == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int e = 0; e < E; e += 4)
          *reinterpret_cast<float4*>(&s_cacc[sub][g * D + dl * E + e]) =
              make_float4(acc[g][e], acc[g][e + 1], acc[g][e + 2], acc[g][e + 3]);
        if (dl == 0) {
          s_cm[sub][g] = m[g];
          s_cl[sub][g] = l[g];
        }
      }
    }
    __syncthreads();
    for (int o = threadIdx.x; o < G * D; o += 64 * SPLIT) {
      const int g = o / D, d = o - g * D;
      float M = s_cm[0][g];
#pragma unroll
      for (int x = 1; x < SPLIT; ++x) M = fmaxf(M, s_cm[x][g]);
      float ls = 0.0f, v = 0.0f;
#pragma unroll
      for (int x = 0; x < SPLIT; ++x) {
        const float mx = s_cm[x][g];
        const float wx = (mx == -INFINITY) ? 0.0f : exp2f(mx - M);
        ls = fmaf(wx, s_cl[x][g], ls);
        v = fmaf(wx, s_cacc[x][o], v);
      }
      if (nparts == 1) {
        out[(head0 + g) * D + d] = ls > 0.0f ? v / ls : 0.0f;
      } else {
        const int64_t row = (head0 + g) * max_parts + part;
        part_acc[row * D + d] = v;
        if (d == 0) {
          part_ml[row * 2 + 0] = M;
          part_ml[row * 2 + 1] = ls;
        }
      }
    }
  }
}

// grid = (num_q_heads, num_seqs), one workgroup of kMergeWaves waves per
// (query head, sequence).  All threads take the partition maxima and the
// weights 2^(m_p - M) (kept in LDS); then lane l of a wave reads float4 c =
// l % (D/4) of partition rows p = l / (D/4) + ..., so one wave instruction
// covers 64 / (D/4) partitions (2 for D = 128) and the kMergeWaves waves
// split the partitions; per-row sums meet through shuffles and LDS.
constexpr int kMergeWaves = 4;

template <int D>
__global__ __launch_bounds__(64 * kMergeWaves) void decode_merge_kernel(
    float* __restrict__ out, const float* __restrict__ part_acc,
    const float* __restrict__ part_ml, const int32_t* __restrict__ ctx_lens, int ctx_cap,
    int num_q_heads, int P, int max_parts) {
  constexpr int NT = 64 * kMergeWaves;
  constexpr int V4 = D / 4;        // float4 per partition row
  constexpr int RPW = 64 / V4;     // partition rows per wave instruction
  extern __shared__ float s_w[];   // max_parts weights (dynamic LDS)
  __shared__ float s_red[kMergeWaves];
  __shared__ __align__(16) float s_acc[kMergeWaves][D];
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  int L = ctx_lens[b];
  L = L < 0 ? 0 : (L > ctx_cap ? ctx_cap : L);
  const int np = (L + P - 1) / P;
  if (np <= 1) return;
  const int64_t row0 = ((int64_t)b * num_q_heads + h) * max_parts;
  const int r = lane / V4, c = lane % V4;
  if (np <= kMergeWaves * RPW) {
    // At most one partition row per lane group: the row's acc and its
    // (m, l) are requested together, so the merge waits on memory once.
    __shared__ float s_den[kMergeWaves];
    const int p = w * RPW + r;
    const bool has = p < np;
    const float4 a = has ? *reinterpret_cast<const float4*>(part_acc + (row0 + p) * D + 4 * c)
                         : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float2 ml = has ? *reinterpret_cast<const float2*>(part_ml + (row0 + p) * 2)
                          : make_float2(-INFINITY, 0.0f);
    float M = wave_max(ml.x);
    if (lane == 0) s_red[w] = M;
    __syncthreads();
    M = s_red[0];
#pragma unroll
    for (int x = 1; x < kMergeWaves; ++x) M = fmaxf(M, s_red[x]);
    const float wgt = (ml.x == -INFINITY || M == -INFINITY) ? 0.0f : exp2f(ml.x - M);
    float4 num = make_float4(wgt * a.x, wgt * a.y, wgt * a.z, wgt * a.w);
    const float den = wave_sum(c == 0 ? wgt * ml.y : 0.0f);  // each row's l once
#pragma unroll
    for (int o = V4; o < 64; o <<= 1) {
      num.x += __shfl_xor(num.x, o);
      num.y += __shfl_xor(num.y, o);
      num.z += __shfl_xor(num.z, o);
      num.w += __shfl_xor(num.w, o);
    }
    if (r == 0) *reinterpret_cast<float4*>(&s_acc[w][4 * c]) = num;
    if (lane == 0) s_den[w] = den;
    __syncthreads();
    float dsum = 0.0f;
#pragma unroll
    for (int x = 0; x < kMergeWaves; ++x) dsum += s_den[x];
    for (int dd = tid; dd < D; dd += NT) {
      float v = 0.0f;
#pragma unroll
      for (int x = 0; x < kMergeWaves; ++x) v += s_acc[x][dd];
      out[((int64_t)b * num_q_heads + h) * D + dd] = dsum > 0.0f ? v / dsum : 0.0f;
    }
    return;
  }
  float M = -INFINITY;
  for (int p = tid; p < np; p += NT) M = fmaxf(M, part_ml[(row0 + p) * 2]);
  M = wave_max(M);
  if (lane == 0) s_red[w] = M;
  __syncthreads();
  M = s_red[0];
#pragma unroll
  for (int x = 1; x < kMergeWaves; ++x) M = fmaxf(M, s_red[x]);
  __syncthreads();
  float den = 0.0f;
  for (int p = tid; p < np; p += NT) {
    const float m = part_ml[(row0 + p) * 2];
    const float wgt = (m == -INFINITY || M == -INFINITY) ? 0.0f : exp2f(m - M);
    s_w[p] = wgt;
    den = fmaf(wgt, part_ml[(row0 + p) * 2 + 1], den);
  }
  den = wave_sum(den);
  if (lane == 0) s_red[w] = den;
  __syncthreads();
  den = 0.0f;
#pragma unroll
  for (int x = 0; x < kMergeWaves; ++x) den += s_red[x];
  // weighted sum of the acc rows
  float4 num = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 4
  for (int p = w * RPW + r; p < np; p += kMergeWaves * RPW) {
    const float wgt = s_w[p];
    const float4 a = *reinterpret_cast<const float4*>(part_acc + (row0 + p) * D + 4 * c);
    num.x = fmaf(wgt, a.x, num.x);
    num.y = fmaf(wgt, a.y, num.y);
    num.z = fmaf(wgt, a.z, num.z);
    num.w = fmaf(wgt, a.w, num.w);
  }
#pragma unroll
  for (int o = V4; o < 64; o <<= 1) {
    num.x += __shfl_xor(num.x, o);
    num.y += __shfl_xor(num.y, o);
    num.z += __shfl_xor(num.z, o);
    num.w += __shfl_xor(num.w, o);
  }
  if (r == 0) *reinterpret_cast<float4*>(&s_acc[w][4 * c]) = num;
  __syncthreads();
  for (int dd = tid; dd < D; dd += NT) {
    float v = 0.0f;
#pragma unroll
    for (int x = 0; x < kMergeWaves; ++x) v += s_acc[x][dd];
    out[((int64_t)b * num_q_heads + h) * D + dd] = den > 0.0f ? v / den : 0.0f;
  }
}

// Merge for calls with at most kMergeRowsMaxParts partitions per sequence
// (max_context <= 8 partitions: configs[2] and most decode batches).  One
// wave per (sequence, query head), four per workgroup, no LDS and no
// barrier: lane l holds float4 c = l % (D/4) of partition rows
// p = l / (D/4) + RPW j, and the rows meet through cross-lane reductions.
// The length and every row the call could have written are requested
// together (rows at or past the sequence's partition count hold stale bytes
// from earlier calls and are removed by selects, never multiplied), so the
// wave waits on memory once.
constexpr int kMergeRowsMaxParts = 8;

// Reduction over the RPW lanes l, l + V4, l + 2 V4, ... (same column c).
template <int V4, bool MAX>
__device__ __forceinline__ float rows_reduce(float x) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  if constexpr (V4 <= 8) x = op(x, dpp<0x128>(x));  // lane l ^ 8 inside a 16-lane row
  if constexpr (V4 <= 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

template <int D>
__global__ __launch_bounds__(256) void decode_merge_rows_kernel(
    float* __restrict__ out, const float* __restrict__ part_acc,
    const float* __restrict__ part_ml, const int32_t* __restrict__ ctx_lens, int ctx_cap,
    int num_q_heads, int P, int max_parts, int n_rows) {
  constexpr int V4 = D / 4, RPW = 64 / V4, J = kMergeRowsMaxParts / RPW;
  static_assert(RPW >= 2 && J >= 1, "head_dim 32, 64 or 128");
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);  // sequence * num_q_heads + head
  if (row >= n_rows) return;
  const int b = row / num_q_heads;
  int L = ctx_lens[b];
  const int r = lane / V4, c = lane % V4;
  const int64_t row0 = (int64_t)row * max_parts;
  float4 a[J];
  float2 ml[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int p = r + RPW * j;
    if (p < max_parts) {
      a[j] = *reinterpret_cast<const float4*>(part_acc + (row0 + p) * D + 4 * c);
      ml[j] = *reinterpret_cast<const float2*>(part_ml + (row0 + p) * 2);
    } else {
      a[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      ml[j] = make_float2(-INFINITY, 0.0f);
    }
  }
  L = L < 0 ? 0 : (L > ctx_cap ? ctx_cap : L);
  const int np = (L + P - 1) / P;
  if (np <= 1) return;  // finished by the partition pass
  float m[J], M = -INFINITY;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    m[j] = r + RPW * j < np ? ml[j].x : -INFINITY;
    M = fmaxf(M, m[j]);
  }
  M = rows_reduce<V4, true>(M);
  float4 num = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float den = 0.0f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const bool use = m[j] != -INFINITY;  // a written row of a partition with a valid token
    const float w = use ? exp2f(m[j] - M) : 0.0f;
    const float4 x = use ? a[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    num.x = fmaf(w, x.x, num.x);
    num.y = fmaf(w, x.y, num.y);
    num.z = fmaf(w, x.z, num.z);
    num.w = fmaf(w, x.w, num.w);
    den = fmaf(w, use ? ml[j].y : 0.0f, den);
  }
  num.x = rows_reduce<V4, false>(num.x);
  num.y = rows_reduce<V4, false>(num.y);
  num.z = rows_reduce<V4, false>(num.z);
  num.w = rows_reduce<V4, false>(num.w);
  den = rows_reduce<V4, false>(den);
  if (r == 0) {
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    *reinterpret_cast<float4*>(out + (int64_t)row * D + 4 * c) =
        den > 0.0f ? make_float4(num.x * inv, num.y * inv, num.z * inv, num.w * inv)
                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
}

// ---- dispatch ----------------------------------------------------------------

constexpr int kBS = 16;
// Tokens per partition, waves per partition (each streams a slice) and the
// register ring depth in 16-byte loads per lane (16-bit / fp32 pools, 1-byte
// pools).
#ifndef RKV_DECODE_P
#define RKV_DECODE_P 640  // 40 blocks; 2.8% faster than 512 at configs[2], 4% for 1-byte pools
#endif
#ifndef RKV_DECODE_SPLIT
#define RKV_DECODE_SPLIT 4
#endif
#ifndef RKV_DECODE_RING_LOADS
#define RKV_DECODE_RING_LOADS 16
#endif
#ifndef RKV_DECODE_RING_LOADS_Q  // 1-byte pools (more registers per tile)
#define RKV_DECODE_RING_LOADS_Q 8
#endif
// bf16 pools at head_dim 128: bytes of unused dynamic LDS per workgroup,
// a knob on how many workgroups share a CU (39 KiB each: four).  With the
// streaming (nontemporal) K/V loads, four per CU beat three (14 KiB of
// padding) by ~2% at configs[2]; with ordinary loads it was the reverse.
#ifndef RKV_DECODE_LDS_PAD_16
#define RKV_DECODE_LDS_PAD_16 0
#endif
// 1-byte pools carry half the bytes per token: their own partition size and
// waves per partition.
#ifndef RKV_DECODE_P_Q
#define RKV_DECODE_P_Q RKV_DECODE_P
#endif
#ifndef RKV_DECODE_SPLIT_Q
#define RKV_DECODE_SPLIT_Q RKV_DECODE_SPLIT
#endif
constexpr int kP = RKV_DECODE_P;
constexpr int kPQ = RKV_DECODE_P_Q;
template <typename T>
constexpr int part_of() { return sizeof(T) == 1 ? kPQ : kP; }
template <typename T>
constexpr int split_of() { return sizeof(T) == 1 ? RKV_DECODE_SPLIT_Q : RKV_DECODE_SPLIT; }

// Partition sizes.  A call's partition size P (tokens) is any multiple of
// 16 * SPLIT up to the build's largest (640); its waves stream
// tw = P / (16 * SPLIT) tiles each.  The kernels are built for two slice
// lengths: the largest, and for 16-bit and fp32 pools also 512 tokens, so
// that a caller asking for 512-token partitions runs them without masked
// slots; other sizes run on the smallest build that holds them, the extra
// slots masked.
// bf16 pools also have two builds of 8-wave workgroups: 768 tokens (a
// 96-token slice, 6 tiles, per wave) and 1280 tokens (10 tiles per wave, the
// 640-token build's slice); requests that are multiples of 128 above 640 run
// on them.  Measured in one process against the 4-wave
// 640-token build (us per call): configs[2] (64 sequences, contexts
// U[512, 4096]) 109.0 -> 106.7 at 768 (122.8 at 1280: too few workgroups);
// 256 x U[1, 8192] 769.3 -> 736.9 at 1280; 64 x U[8192, 16384] 547.0 ->
// 526.5; 32 x U[12288, 24576] 403.4 -> 387.1; configs[3] (8 x U[16384,
// 65536]) 221.2 -> 214.2.  Fewer partitions per sequence mean fewer split-K
// partials and a cheaper merge.
// They pay off only with enough work: at 8 x U[512, 4096] 768 was 5% slower
// than 640, at 4 x U[16384, 32768] 1280 was 10% slower, and for 8 query
// heads per KV head (more registers, two waves per SIMD) both were slower
// (64 x U[512, 4096]: 125 -> 158 us), as for head_dim 64.
// Defaults: the split entry points (rkv_decode_attention_partitions /
// _merge, which take no KV-head count) and fp32 / 1-byte pools use 640;
// rkv_decode_attention picks by the call's shape (shape_part).
constexpr int kSmallP = 512;
static_assert(kSmallP <= kP && kSmallP % (16 * RKV_DECODE_SPLIT) == 0, "small partition build");
static_assert(kSmallP <= kPQ && kSmallP % (16 * RKV_DECODE_SPLIT_Q) == 0,
              "small partition build of the 1-byte pools");
constexpr int kWideSplit = 8;
constexpr int kWideP1 = 768, kWideP2 = 1280;
static_assert(kWideP1 % (16 * kWideSplit) == 0 && kWideP2 % (16 * kWideSplit) == 0 &&
                  kWideP1 > kP,
              "wide partition builds");

inline bool one_byte(int dtype) { return dtype == RKV_I8 || dtype == RKV_FP8; }

int default_part(int dtype, int /*max_context*/) { return one_byte(dtype) ? kPQ : kP; }

// The partition size rkv_decode_attention uses when the caller leaves it to
// the library: for bf16 pools with head_dim 128 and at most 4 query heads
// per KV head, 1280 when the call holds work for at least 1,200 such
// partitions over all KV heads (contexts taken as uniform up to cap), else
// 768 when it holds work for 1,000 of those, else 640 when it holds work for
// 800 partitions of 512, else 512 (the measurements above: configs[2] 768,
// configs[3] and 256 x U[1, 8192] 1280; and, us per call at 512 / 640 /
// 768 over U[512, 4096] contexts, 32 layers back to back: 8 sequences x 8
// KV heads 19.5 / 22.4 / 24.3, 64 x 1 (configs[2]'s share of one GPU of 8
// by KV heads) 23.8 / 24.5 / 25.9, 16 x 8 33.4 / 38.9 / 35.9, 64 x 2 36.9 /
// 41.4 / 40.7, 24 x 8 42.4 / 43.5 / 43.8, 32 x 8 56.4 / 56.5 / 55.7, 64 x 4
// 60.8 / 58.9 / 64.6, 48 x 8 82.8 / 81.7 / 81.3).
// The 512-token tier holds for fp32 pools and every head shape: 512 / 640
// us at 8 and 16 sequences x 8 KV heads, G = 8: 21.9 / 23.7, 32.0 / 37.1;
// head_dim 64: 13.5 / 15.1, 20.6 / 23.6; fp32 pools: 31.8 / 37.3, 58.9 /
// 69.0; at 32 and 64 sequences even or 640 ahead (G = 8 at 64: 121.6 /
// 116.3).  1-byte pools take it up to twice the work (int8, contexts U[512,
// 4096], 512 / 640: 8 sequences 13.4 / 15.2, 16 sequences 21.0 / 24.2, 32
// sequences 33.0 / 33.8, 64 sequences 66.5 / 64.2; 64 x 1 KV head 16.0 /
// 16.4).
int shape_part(int dtype, int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
               int cap) {
  if (num_kv_heads <= 0 || num_seqs <= 0 || cap <= 0) return default_part(dtype, cap);
  const double work = (double)num_kv_heads * num_seqs * (0.5 * cap);  // KV-head tokens
  if (work < (one_byte(dtype) ? 1600.0 : 800.0) * kSmallP) return kSmallP;
  if (one_byte(dtype)) return default_part(dtype, cap);
  if (dtype != RKV_BF16 || head_dim != 128 || num_q_heads % num_kv_heads != 0 ||
      num_q_heads / num_kv_heads > 4)
    return default_part(dtype, cap);
  if (work >= 1200.0 * kWideP2) return kWideP2;
  if (work >= 1000.0 * kWideP1) return kWideP1;
  return kP;
}

// The partition size a call uses: the request when it is > 0 (a multiple of
// 16 * SPLIT up to the largest 4-wave build, or for bf16 pools a multiple of
// 128 up to 1280), else the default; a negative status for an unsupported
// request.
int resolve_part(int requested, int dtype, int max_context) {
  if (requested <= 0) return default_part(dtype, max_context);
  const int split = one_byte(dtype) ? RKV_DECODE_SPLIT_Q : RKV_DECODE_SPLIT;
  const int maxp = one_byte(dtype) ? kPQ : kP;
  if (requested % (16 * split) == 0 && requested <= maxp) return requested;
  if (dtype == RKV_BF16 && requested > maxp && requested <= kWideP2 &&
      requested % (16 * kWideSplit) == 0)
    return requested;
  return RKV_ERR_UNSUPPORTED;
}

struct Launch {
  int nw = 0;
  void (*kernel)(float*, float*, float*, const float*, const void*, const void*, const float*,
                 const float*, const int32_t*, int, const int32_t*, int, int, int64_t, float,
                 int, int, const float*, const float*) = nullptr;
};

// Ring depth: RKV_DECODE_RING_LOADS 16-byte loads per lane in flight, at most
// every tile of the wave's slice.
template <typename T, int D, int NTILE, int SPLIT>
constexpr int ring_for() {
  constexpr int nl = kBS / (64 / (D / Traits<T>::E));
  constexpr int r = (sizeof(T) == 1 ? RKV_DECODE_RING_LOADS_Q : RKV_DECODE_RING_LOADS) / nl;
  constexpr int nt = 2 * NTILE / SPLIT;
  return r < 1 ? 1 : (r > nt ? nt : r);
}

template <typename T, int D, int G, int FMT, int NTILE, int SPLIT = split_of<T>()>
Launch make_launch(bool append) {
  Launch l;
  l.nw = SPLIT;
  if constexpr (FMT == RKV_BF16 || FMT == RKV_I8 || FMT == RKV_FP8) {  // fused append builds
    if (append) {
      l.kernel = &decode_stream_kernel<T, D, G, kBS, NTILE, ring_for<T, D, NTILE, SPLIT>(),
                                       SPLIT, FMT, true>;
      return l;
    }
  } else if (append) {
    return Launch{};
  }
  l.kernel = &decode_stream_kernel<T, D, G, kBS, NTILE, ring_for<T, D, NTILE, SPLIT>(), SPLIT,
                                   FMT>;
  return l;
}

// The build for partitions of P tokens: above the largest 4-wave build (bf16
// pools), the smallest 8-wave build that holds them; else the 512-token
// build when it holds them, else the largest.
template <typename T, int D, int G, int FMT>
Launch pick_p(int P, bool append) {
  if constexpr (FMT == RKV_BF16) {
    if (P > kP) {
      if (P <= kWideP1) return make_launch<T, D, G, FMT, kWideP1 / kBS, kWideSplit>(append);
      return make_launch<T, D, G, FMT, kWideP2 / kBS, kWideSplit>(append);
    }
  }
  if constexpr (kSmallP < part_of<T>()) {
    if (P <= kSmallP) return make_launch<T, D, G, FMT, kSmallP / kBS>(append);
  }
  return make_launch<T, D, G, FMT, part_of<T>() / kBS>(append);
}

template <typename T, int D, int FMT>
Launch pick_g(int G, int P, bool append) {
  switch (G) {
    case 1: return pick_p<T, D, 1, FMT>(P, append);
    case 2: return pick_p<T, D, 2, FMT>(P, append);
    case 4: return pick_p<T, D, 4, FMT>(P, append);
    case 8: return pick_p<T, D, 8, FMT>(P, append);
    default: return Launch{};
  }
}

// 16-bit and fp32 pools: head_dim 32, 64, 128; 1-byte pools: 64, 128.
template <typename T, int FMT>
Launch pick_d(int D, int G, int P, bool append) {
  switch (D) {
    case 32:
      if constexpr (sizeof(T) == 1) return Launch{};
      else return pick_g<T, 32, FMT>(G, P, append);
    case 64: return pick_g<T, 64, FMT>(G, P, append);
    case 128: return pick_g<T, 128, FMT>(G, P, append);
    default: return Launch{};
  }
}

Launch pick(int dtype, int D, int G, int P, bool append) {
  switch (dtype) {
    case RKV_F32: return pick_d<float, RKV_F32>(D, G, P, append);
    case RKV_BF16: return pick_d<uint16_t, RKV_BF16>(D, G, P, append);
    case RKV_I8: return pick_d<uint8_t, RKV_I8>(D, G, P, append);
    case RKV_FP8: return pick_d<uint8_t, RKV_FP8>(D, G, P, append);
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
  const float* k_scale = nullptr;  // 1-byte pools: [num_blocks][Hkv][block_size] fp32
  const float* v_scale = nullptr;
  const float* k_new = nullptr;  // fused append (bf16 pools): [num_seqs][Hkv][D] fp32
  const float* v_new = nullptr;
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

int validate(const DecodeArgs& a, int& max_parts, int& P) {
  if (a.num_seqs < 0 || a.max_blocks_per_seq < 0 || a.num_blocks < 0)
    return fail(RKV_ERR_INVALID_ARG, "negative size argument");
  if (a.num_q_heads <= 0 || a.num_kv_heads <= 0 || a.num_q_heads % a.num_kv_heads)
    return fail(RKV_ERR_INVALID_ARG, "num_q_heads must be a positive multiple of num_kv_heads");
  const bool q8 = a.dtype == RKV_I8 || a.dtype == RKV_FP8;
  if (a.dtype != RKV_F32 && a.dtype != RKV_BF16 && !q8)
    return fail(RKV_ERR_INVALID_ARG, "dtype must be RKV_F32, RKV_BF16, RKV_I8 or RKV_FP8");
  if (q8 && a.head_dim == 32)
    return fail(RKV_ERR_UNSUPPORTED, "1-byte pools: head_dim must be 64 or 128");
  if (a.block_size != kBS) return fail(RKV_ERR_UNSUPPORTED, "block_size must be 16");
  if (a.head_dim != 32 && a.head_dim != 64 && a.head_dim != 128)
    return fail(RKV_ERR_UNSUPPORTED, "head_dim must be 32, 64 or 128");
  const int G = a.num_q_heads / a.num_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return fail(RKV_ERR_UNSUPPORTED, "num_q_heads / num_kv_heads must be 1, 2, 4 or 8");
  P = resolve_part(a.partition_size, a.dtype, a.max_context);
  if (P < 0)
    return fail(RKV_ERR_UNSUPPORTED,
                "partition_size must be a multiple of 64 tokens up to 640, for bf16 pools also a "
                "multiple of 128 up to 1280 (or <= 0 for the default)");
  if (a.num_seqs > 65535 || a.num_kv_heads > 65535)
    return fail(RKV_ERR_INVALID_ARG, "num_seqs and num_kv_heads must be <= 65535");
  if (a.max_context < 0) return fail(RKV_ERR_INVALID_ARG, "max_context must be >= 0");
  if (a.num_blocks < 1) return fail(RKV_ERR_INVALID_ARG, "num_blocks must be >= 1");
  const int cap = ctx_cap_of(a.max_context, a.max_blocks_per_seq, a.block_size);
  max_parts = cap <= 0 ? 1 : (cap + P - 1) / P;
  if (max_parts > kMaxMergeParts)
    return fail(RKV_ERR_UNSUPPORTED, "max_context / partition size above 4096 partitions");
  if (a.num_seqs == 0) return RKV_OK;
  if (!a.out || !a.q || !a.k_pool || !a.v_pool || !a.block_tables || !a.ctx_lens)
    return fail(RKV_ERR_INVALID_ARG, "null pointer argument");
  if (q8 && (!a.k_scale || !a.v_scale))
    return fail(RKV_ERR_INVALID_ARG,
                "1-byte pools need their scale pools (rkv_decode_attention_q)");
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

int launch_partitions(const DecodeArgs& a, int max_parts, int P) {
  const int G = a.num_q_heads / a.num_kv_heads;

  Launch l = pick(a.dtype, a.head_dim, G, P, a.k_new != nullptr);
  if (!l.kernel) return fail(RKV_ERR_UNSUPPORTED, "no decode kernel for this shape");
  float *acc = nullptr, *ml = nullptr;
  if (max_parts > 1) split_ws(a.workspace, a.num_seqs, a.num_q_heads, a.head_dim, max_parts, acc, ml);
  const int cap = ctx_cap_of(a.max_context, a.max_blocks_per_seq, a.block_size);
  // KV-head major: the Hkv workgroups of one (partition, sequence) are adjacent
  const dim3 grid((unsigned)a.num_kv_heads, (unsigned)max_parts, (unsigned)a.num_seqs);
  const size_t pad = (a.dtype == RKV_BF16 && a.head_dim == 128) ? RKV_DECODE_LDS_PAD_16 : 0;
  hipLaunchKernelGGL(l.kernel, grid, dim3(l.nw * 64), pad, a.stream, a.out, acc, ml, a.q, a.k_pool,
                     a.v_pool, a.k_scale, a.v_scale, a.block_tables, a.max_blocks_per_seq,
                     a.ctx_lens, cap,
                     a.num_kv_heads, a.num_blocks, a.scale * kLog2e, max_parts,
                     P / (kBS * l.nw), a.k_new, a.v_new);
  return check_launch("decode_stream_kernel");
}

int launch_merge(float* out, const int32_t* ctx_lens, int num_seqs, int num_q_heads, int head_dim,
                 int cap, int P, int max_parts, void* ws, hipStream_t stream) {
  if (max_parts <= 1 || num_seqs == 0) return RKV_OK;
  float *acc = nullptr, *ml = nullptr;
  split_ws(ws, num_seqs, num_q_heads, head_dim, max_parts, acc, ml);
  if (max_parts <= kMergeRowsMaxParts && (int64_t)num_seqs * num_q_heads <= (1 << 28)) {
    const int n_rows = num_seqs * num_q_heads;
    const unsigned nwg = (unsigned)((n_rows + 3) / 4);
    switch (head_dim) {
      case 32:
        decode_merge_rows_kernel<32><<<nwg, 256, 0, stream>>>(out, acc, ml, ctx_lens, cap,
                                                              num_q_heads, P, max_parts, n_rows);
        break;
      case 64:
        decode_merge_rows_kernel<64><<<nwg, 256, 0, stream>>>(out, acc, ml, ctx_lens, cap,
                                                              num_q_heads, P, max_parts, n_rows);
        break;
      default:
        decode_merge_rows_kernel<128><<<nwg, 256, 0, stream>>>(out, acc, ml, ctx_lens, cap,
                                                               num_q_heads, P, max_parts, n_rows);
        break;
    }
    return check_launch("decode_merge_rows_kernel");
  }
  dim3 grid((unsigned)num_q_heads, (unsigned)num_seqs);
  const size_t lds = (size_t)max_parts * sizeof(float);
  switch (head_dim) {
    case 32:
      decode_merge_kernel<32><<<grid, 64 * kMergeWaves, lds, stream>>>(out, acc, ml, ctx_lens, cap, num_q_heads,
                                                       P, max_parts);
      break;
    case 64:
      decode_merge_kernel<64><<<grid, 64 * kMergeWaves, lds, stream>>>(out, acc, ml, ctx_lens, cap, num_q_heads,
                                                       P, max_parts);
      break;
    default:
      decode_merge_kernel<128><<<grid, 64 * kMergeWaves, lds, stream>>>(out, acc, ml, ctx_lens, cap, num_q_heads,
                                                        P, max_parts);
      break;
  }
  return check_launch("decode_merge_kernel");
}

}  // namespace
}  // namespace rkv

using namespace rkv;

extern "C" size_t rkv_decode_workspace_bytes(int num_seqs, int num_q_heads, int head_dim,
                                             int max_context, int partition_size) {
  if (num_seqs <= 0 || num_q_heads <= 0 || head_dim <= 0 || max_context <= 0) return 0;
  // a given partition size, else the smallest size a call picks by itself
  // (the 512-token build's, for small bf16 calls): enough for every pool
  // dtype and shape
  const int dflt = std::min({kSmallP, default_part(RKV_BF16, max_context),
                             default_part(RKV_I8, max_context)});
  const int P = partition_size > 0 ? partition_size : dflt;
  const int max_parts = (max_context + P - 1) / P;
  return ws_bytes(num_seqs, num_q_heads, head_dim, max_parts);
}

extern "C" int rkv_decode_partition_size(int partition_size, int head_dim, int dtype,
                                         int max_context) {
  clear_error();
  (void)head_dim;
  if (dtype != RKV_F32 && dtype != RKV_BF16 && !one_byte(dtype))
    return fail(RKV_ERR_INVALID_ARG, "dtype must be RKV_F32, RKV_BF16, RKV_I8 or RKV_FP8");
  const int P = resolve_part(partition_size, dtype, max_context);
  if (P < 0)
    return fail(P, "partition_size must be a multiple of 64 tokens up to 640, for bf16 pools also "
                   "a multiple of 128 up to 1280 (or <= 0)");
  return P;
}

extern "C" int rkv_decode_partition_size_for(int partition_size, int num_seqs, int num_q_heads,
                                             int num_kv_heads, int head_dim, int dtype,
                                             int max_context) {
  clear_error();
  if (dtype != RKV_F32 && dtype != RKV_BF16 && !one_byte(dtype))
    return fail(RKV_ERR_INVALID_ARG, "dtype must be RKV_F32, RKV_BF16, RKV_I8 or RKV_FP8");
  if (partition_size <= 0)
    return shape_part(dtype, num_seqs, num_q_heads, num_kv_heads, head_dim,
                      max_context < 0 ? 0 : max_context);
  const int P = resolve_part(partition_size, dtype, max_context);
  if (P < 0)
    return fail(P, "partition_size must be a multiple of 64 tokens up to 640, for bf16 pools also "
                   "a multiple of 128 up to 1280 (or <= 0)");
  return P;
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
  int max_parts = 1, P = 0;
  if (int rc = validate(a, max_parts, P)) return rc;
  if (num_seqs == 0) return RKV_OK;
  return launch_partitions(a, max_parts, P);
}

extern "C" int rkv_decode_attention_merge(float* out, const int32_t* ctx_lens,
                                          int max_blocks_per_seq, int num_seqs, int num_q_heads,
                                          int head_dim, int block_size, int max_context,
                                          int dtype, int partition_size, const void* workspace,
                                          size_t workspace_bytes, void* stream) {
  clear_error();
  if (num_seqs < 0 || num_q_heads <= 0 || max_blocks_per_seq < 0 || max_context < 0)
    return fail(RKV_ERR_INVALID_ARG, "bad size argument");
  if (block_size != kBS) return fail(RKV_ERR_UNSUPPORTED, "block_size must be 16");
  if (head_dim != 32 && head_dim != 64 && head_dim != 128)
    return fail(RKV_ERR_UNSUPPORTED, "head_dim must be 32, 64 or 128");
  const int P = resolve_part(partition_size, dtype, max_context);
  if (P < 0)
    return fail(RKV_ERR_UNSUPPORTED,
                "partition_size must be a multiple of 64 tokens up to 640, for bf16 pools also a "
                "multiple of 128 up to 1280 (or <= 0 for the default)");
  if (num_seqs > 65535 || num_q_heads > 65535)
    return fail(RKV_ERR_INVALID_ARG, "num_seqs and num_q_heads must be <= 65535");
  const int cap = ctx_cap_of(max_context, max_blocks_per_seq, block_size);
  const int max_parts = cap <= 0 ? 1 : (cap + P - 1) / P;
  if (max_parts > kMaxMergeParts)
    return fail(RKV_ERR_UNSUPPORTED, "max_context / partition size above 4096 partitions");
  if (max_parts <= 1 || num_seqs == 0) return RKV_OK;
  if (!out || !ctx_lens) return fail(RKV_ERR_INVALID_ARG, "null pointer argument");
  const size_t need = ws_bytes(num_seqs, num_q_heads, head_dim, max_parts);
  if (!workspace || workspace_bytes < need)
    return fail(RKV_ERR_WORKSPACE, "workspace missing or smaller than rkv_decode_workspace_bytes()");
  return launch_merge(out, ctx_lens, num_seqs, num_q_heads, head_dim, cap, P, max_parts,
                      const_cast<void*>(workspace), static_cast<hipStream_t>(stream));
}

extern "C" int rkv_decode_attention(float* out, const float* q, const void* k_pool,
                                    const void* v_pool, const int32_t* block_tables,
                                    int max_blocks_per_seq, const int32_t* ctx_lens, int num_seqs,
                                    int num_q_heads, int num_kv_heads, int head_dim,
                                    int block_size, int64_t num_blocks, int max_context,
                                    float scale, int dtype, int partition_size, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  // both passes take the same explicit partition size: the request, or the
  // size shape_part picks for this call
  const int P =
      partition_size > 0
          ? partition_size
          : shape_part(dtype, num_seqs, num_q_heads, num_kv_heads, head_dim,
                       ctx_cap_of(max_context < 0 ? 0 : max_context,
                                  max_blocks_per_seq < 0 ? 0 : max_blocks_per_seq, block_size));
  int rc = rkv_decode_attention_partitions(out, q, k_pool, v_pool, block_tables,
                                           max_blocks_per_seq, ctx_lens, num_seqs, num_q_heads,
                                           num_kv_heads, head_dim, block_size, num_blocks,
                                           max_context, scale, dtype, P, workspace,
                                           workspace_bytes, stream);
  if (rc) return rc;
  return rkv_decode_attention_merge(out, ctx_lens, max_blocks_per_seq, num_seqs, num_q_heads,
                                    head_dim, block_size, max_context, dtype, P, workspace,
                                    workspace_bytes, stream);
}

// Decode with the step's K/V append fused in (bf16 pools).  In the partition
// that holds position ctx_lens[b] - 1, the wave whose slice covers it stores
// the rounded new row into the pools from the lanes whose ring loads read
// that row, waits for the stores (vmcnt(0), that wave only), and then
// streams its tiles as usual, reading the new row back with them; so the
// result equals rkv_append of those rows followed by rkv_decode_attention,
// bit for bit, in one launch fewer.
extern "C" int rkv_decode_attention_append(
    float* out, const float* q, void* k_pool, void* v_pool, const float* k_new,
    const float* v_new, const int32_t* block_tables, int max_blocks_per_seq,
    const int32_t* ctx_lens, int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
    int block_size, int64_t num_blocks, int max_context, float scale, int dtype,
    int partition_size, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (dtype != RKV_BF16)
    return fail(RKV_ERR_UNSUPPORTED,
                "rkv_decode_attention_append: RKV_BF16 pools (1-byte pools: "
                "rkv_decode_attention_append_q)");
  if (num_seqs > 0 && (!k_new || !v_new))
    return fail(RKV_ERR_INVALID_ARG, "null pointer argument");
  if (num_seqs > 0 && (!aligned16(k_new) || !aligned16(v_new)))
    return fail(RKV_ERR_INVALID_ARG, "k_new and v_new must be 16-byte aligned");
  const int P =
      partition_size > 0
          ? partition_size
          : shape_part(dtype, num_seqs, num_q_heads, num_kv_heads, head_dim,
                       ctx_cap_of(max_context < 0 ? 0 : max_context,
                                  max_blocks_per_seq < 0 ? 0 : max_blocks_per_seq, block_size));
  DecodeArgs a{out, q, k_pool, v_pool, block_tables, max_blocks_per_seq, ctx_lens, num_seqs,
               num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, max_context, scale,
               dtype, P, workspace, workspace_bytes, static_cast<hipStream_t>(stream)};
  a.k_new = k_new;
  a.v_new = v_new;
  int max_parts = 1, P2 = 0;
  if (int rc = validate(a, max_parts, P2)) return rc;
  if (num_seqs == 0) return RKV_OK;
  if (int rc = launch_partitions(a, max_parts, P2)) return rc;
  return launch_merge(out, ctx_lens, num_seqs, num_q_heads, head_dim,
                      ctx_cap_of(max_context, max_blocks_per_seq, block_size), P2, max_parts,
                      workspace, a.stream);
}

// rkv_decode_attention_append for 1-byte pools: the new rows quantized as
// rkv_append_q quantizes them.
extern "C" int rkv_decode_attention_append_q(
    float* out, const float* q, void* k_pool, void* v_pool, float* k_scale, float* v_scale,
    const float* k_new, const float* v_new, const int32_t* block_tables, int max_blocks_per_seq,
    const int32_t* ctx_lens, int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
    int block_size, int64_t num_blocks, int max_context, float scale, int dtype,
    int partition_size, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (dtype != RKV_I8 && dtype != RKV_FP8)
    return fail(RKV_ERR_INVALID_ARG,
                "rkv_decode_attention_append_q: dtype must be RKV_I8 or RKV_FP8");
  if (num_seqs > 0 && (!k_new || !v_new))
    return fail(RKV_ERR_INVALID_ARG, "null pointer argument");
  if (num_seqs > 0 && (!aligned16(k_new) || !aligned16(v_new)))
    return fail(RKV_ERR_INVALID_ARG, "k_new and v_new must be 16-byte aligned");
  DecodeArgs a{out, q, k_pool, v_pool, block_tables, max_blocks_per_seq, ctx_lens, num_seqs,
               num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, max_context, scale,
               dtype, partition_size, workspace, workspace_bytes,
               static_cast<hipStream_t>(stream), k_scale, v_scale};
  a.k_new = k_new;
  a.v_new = v_new;
  int max_parts = 1, P = 0;
  if (int rc = validate(a, max_parts, P)) return rc;
  if (num_seqs == 0) return RKV_OK;
  if (int rc = launch_partitions(a, max_parts, P)) return rc;
  return launch_merge(out, ctx_lens, num_seqs, num_q_heads, head_dim,
                      ctx_cap_of(max_context, max_blocks_per_seq, block_size), P, max_parts,
                      workspace, a.stream);
}

// ---- the entry point that allocates nothing -----------------------------------
// Callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc) get the split-K
// partials from a file-scope device array instead of a workspace argument.
// Every GPU the library runs on holds its own copy until the process ends.
// Its address on a device comes from hipGetSymbolAddress (the array's name in
// host code is only a stand-in for the symbol), taken once per device with
// that device current and kept.
constexpr size_t kScratchBytes = size_t(16) << 20;  // 16 MiB
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The scratch array's device address on the device that owns `stream`.
int scratch_for(hipStream_t stream, void** ptr) {
  int dev = -1;
  if (stream) {
    if (hipStreamGetDevice(stream, &dev) != hipSuccess)
      return fail(RKV_ERR_HIP, "rkv_decode_attention_noalloc: hipStreamGetDevice failed");
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return fail(RKV_ERR_HIP, "rkv_decode_attention_noalloc: hipGetDevice failed");
  }
  if (dev < 0 || dev >= kMaxDevices)
    return fail(RKV_ERR_UNSUPPORTED, "rkv_decode_attention_noalloc: device index above 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess)
      return fail(RKV_ERR_HIP, "rkv_decode_attention_noalloc: hipGetDevice failed");
    if (cur != dev && hipSetDevice(dev) != hipSuccess)
      return fail(RKV_ERR_HIP, "rkv_decode_attention_noalloc: hipSetDevice failed");
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p)
      return fail(RKV_ERR_HIP, std::string("rkv_decode_attention_noalloc: hipGetSymbolAddress: ") +
                                   hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return RKV_OK;
}
}  // namespace

extern "C" size_t rkv_decode_noalloc_max_bytes(void) { return kScratchBytes; }

extern "C" int rkv_decode_attention_noalloc(float* out, const float* q, const void* k_pool,
                                            const void* v_pool, const int32_t* block_tables,
                                            int max_blocks_per_seq, const int32_t* ctx_lens,
                                            int num_seqs, int num_q_heads, int num_kv_heads,
                                            int head_dim, int block_size, int64_t num_blocks,
                                            int max_context, float scale, int dtype,
                                            int partition_size, void* stream) {
  clear_error();
  const int cap = ctx_cap_of(max_context < 0 ? 0 : max_context, max_blocks_per_seq < 0 ? 0 : max_blocks_per_seq,
                             block_size);
  // the size rkv_decode_attention will use (the request, or its shape's pick)
  const int P = partition_size > 0
                    ? resolve_part(partition_size, dtype, max_context)
                    : shape_part(dtype, num_seqs, num_q_heads, num_kv_heads, head_dim, cap);
  if (P < 0)
    return fail(RKV_ERR_UNSUPPORTED,
                "partition_size must be a multiple of 64 tokens up to 640, for bf16 pools also a "
                "multiple of 128 up to 1280 (or <= 0 for the default)");
  const int max_parts = cap <= 0 ? 1 : (cap + P - 1) / P;
  const size_t need = (num_seqs > 0 && num_q_heads > 0 && head_dim > 0)
                          ? ws_bytes(num_seqs, num_q_heads, head_dim, max_parts)
                          : 0;
  if (need > kScratchBytes)
    return fail(RKV_ERR_WORKSPACE,
                "rkv_decode_attention_noalloc: split-K partials need " + std::to_string(need) +
                    " bytes, above the 16 MiB scratch (use rkv_decode_attention with a workspace)");
  void* ws = nullptr;
  if (need > 0)
    if (int rc = scratch_for(static_cast<hipStream_t>(stream), &ws)) return rc;
  return rkv_decode_attention(out, q, k_pool, v_pool, block_tables, max_blocks_per_seq, ctx_lens,
                              num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                              num_blocks, max_context, scale, dtype, P, ws,
                              need > 0 ? kScratchBytes : 0, stream);
}

extern "C" int rkv_decode_attention_q(float* out, const float* q, const void* k_pool,
                                      const void* v_pool, const float* k_scale,
                                      const float* v_scale, const int32_t* block_tables,
                                      int max_blocks_per_seq, const int32_t* ctx_lens,
                                      int num_seqs, int num_q_heads, int num_kv_heads,
                                      int head_dim, int block_size, int64_t num_blocks,
                                      int max_context, float scale, int dtype,
                                      int partition_size, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  clear_error();
  if (dtype != RKV_I8 && dtype != RKV_FP8)
    return fail(RKV_ERR_INVALID_ARG, "rkv_decode_attention_q: dtype must be RKV_I8 or RKV_FP8");
  DecodeArgs a{out, q, k_pool, v_pool, block_tables, max_blocks_per_seq, ctx_lens, num_seqs,
               num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, max_context, scale,
               dtype, partition_size, workspace, workspace_bytes,
               static_cast<hipStream_t>(stream), k_scale, v_scale};
  int max_parts = 1, P = 0;
  if (int rc = validate(a, max_parts, P)) return rc;
  if (num_seqs == 0) return RKV_OK;
  if (int rc = launch_partitions(a, max_parts, P)) return rc;
  const int cap = ctx_cap_of(max_context, max_blocks_per_seq, block_size);
  return launch_merge(out, ctx_lens, num_seqs, num_q_heads, head_dim, cap, P, max_parts,
                      workspace, a.stream);
}
