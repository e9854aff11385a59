// kv_copy.hip -- KV append (scatter into pages), gather (pages -> contiguous
// KVCache layout) and block copy (compaction) for gfx950.
//
// All three are HBM-streaming copies.  Every lane moves 16 bytes per access
// (global_load/store_dwordx4), consecutive lanes touch consecutive 16-byte
// chunks of one (block, head) tile, so each wave moves 1 KiB contiguous
// bytes per instruction.  No LDS: there is no reuse to stage.
#include "common.hpp"

#include <type_traits>

namespace rkv {
namespace {

// Load / store policy: 1 = nontemporal (streaming) hint.  Measured on
// configs[1]-sized calls (65,536-block pools, GB/s of algorithmic bytes):
//   gather bf16 -> bf16: plain 5155, nt loads 5387, nt stores 5705, both 6066
//   gather bf16 -> fp32, when a lane stored 8 floats as two 16-byte stores
//                        (no contiguous wave store): plain 4972, nt loads
//                        5197, nt stores 3536; with one lane-contiguous
//                        16-byte store per lane: nt loads 5290-5355, both
//                        6003-6074
//   gather fp32 -> fp32: plain 5344, nt loads 5114, both 5277 (two 16-byte
//                        accesses per lane); lane-contiguous, nt stores
//                        5317-5325, plain 5208-5250
//   copy_blocks: 5082 - 5177 for every policy
// so the gather streams its loads for 16-bit pools and its stores always
// (RKV_GATHER_NT = 0 turns both off), and copy_blocks streams both.
#ifndef RKV_GATHER_NT
#define RKV_GATHER_NT 1
#endif
#ifndef RKV_GATHER_NTS_F32  // nontemporal stores for fp32 outputs as well
#define RKV_GATHER_NTS_F32 1
#endif
#ifndef RKV_COPY_NTL
#define RKV_COPY_NTL 1
#endif
#ifndef RKV_COPY_NTS
#define RKV_COPY_NTS 1
#endif
#ifndef RKV_APPEND_NTL
#define RKV_APPEND_NTL 0
#endif
#ifndef RKV_APPEND_NTS
#define RKV_APPEND_NTS 0
#endif

template <bool NT>
__device__ __forceinline__ uint4 ld16(const void* p) {
  if constexpr (NT) return load_stream(p);
  else return *static_cast<const uint4*>(p);
}

// 16-byte store of the bits of v (any 16-byte trivially copyable type),
// optionally with the nontemporal hint.
template <bool NT = false, typename V>
__device__ __forceinline__ void store16(void* p, const V& v) {
  static_assert(sizeof(V) == 16, "16-byte store");
  if constexpr (NT) __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v), static_cast<u32x4_t*>(p));
  else *static_cast<u32x4_t*>(p) = __builtin_bit_cast(u32x4_t, v);
}

struct alignas(16) F8 {  // 8 floats = 32 bytes
  float4 a, b;
};

template <bool NT = false>
__device__ __forceinline__ F8 load_f8(const float* p) {
  const uint4 a = ld16<NT>(p), b = ld16<NT>(p + 4);
  return F8{__builtin_bit_cast(float4, a), __builtin_bit_cast(float4, b)};
}

template <bool NT = false>
__device__ __forceinline__ void store_f8(float* p, const F8& x) {
  store16<NT>(p, x.a);
  store16<NT>(p + 4, x.b);
}

__device__ __forceinline__ uint4 f8_to_bf16x8(const F8& x) {
  return make_uint4(pack_bf16x2(x.a.x, x.a.y), pack_bf16x2(x.a.z, x.a.w),
                    pack_bf16x2(x.b.x, x.b.y), pack_bf16x2(x.b.z, x.b.w));
}

// ---- append -----------------------------------------------------------------
// grid = (n_tokens, n_layers); each thread moves 8 elements of K and of V.
// The source rows do not depend on the slot, so the first chunk's K/V loads
// are issued before the slot is waited on (straight-line code; the loop for
// further chunks only runs when Hkv * D / 8 exceeds the workgroup).  bs_log2
// is log2(block_size) for a power-of-two block size, else -1 (division).
template <bool BF16>
__global__ __launch_bounds__(256) void append_kernel(
    void* __restrict__ k_pool, void* __restrict__ v_pool, int64_t pool_layer_stride,
    const float* __restrict__ k_new, const float* __restrict__ v_new, int64_t src_layer_stride,
    int64_t src_tok_stride, int64_t src_head_stride, const int64_t* __restrict__ slot_mapping,
    int num_kv_heads, int head_dim, int block_size, int bs_log2, int64_t num_slots) {
  const int t = blockIdx.x, layer = blockIdx.y;
  const int chunks = head_dim >> 3;
  const int units = num_kv_heads * chunks;
  const int64_t src0 = layer * src_layer_stride + t * src_tok_stride;
  auto src_of = [&](int u) {
    const int h = u / chunks, c = u - h * chunks;
    return src0 + h * src_head_stride + c * 8;
  };
  auto put = [&](int u, int64_t blk, int64_t row, const F8& k, const F8& v) {
    const int h = u / chunks, c = u - h * chunks;
    const int64_t dst =
        layer * pool_layer_stride + ((blk * num_kv_heads + h) * block_size + row) * head_dim + c * 8;
    if constexpr (BF16) {
      store16<RKV_APPEND_NTS>(static_cast<uint16_t*>(k_pool) + dst, f8_to_bf16x8(k));
      store16<RKV_APPEND_NTS>(static_cast<uint16_t*>(v_pool) + dst, f8_to_bf16x8(v));
    } else {
      store_f8<RKV_APPEND_NTS>(static_cast<float*>(k_pool) + dst, k);
      store_f8<RKV_APPEND_NTS>(static_cast<float*>(v_pool) + dst, v);
    }
  };
  const int u0 = threadIdx.x;
  F8 k0, v0;
  if (u0 < units) {
    k0 = load_f8<RKV_APPEND_NTL>(k_new + src_of(u0));
    v0 = load_f8<RKV_APPEND_NTL>(v_new + src_of(u0));
  }
  const int64_t slot = slot_mapping[t];
  if (slot < 0 || slot >= num_slots) return;  // padding or out-of-range slot
  const int64_t blk = bs_log2 >= 0 ? slot >> bs_log2 : slot / block_size;
  const int64_t row = slot - blk * block_size;
  if (u0 < units) put(u0, blk, row, k0, v0);
  for (int u = u0 + blockDim.x; u < units; u += blockDim.x) {
    const F8 k = load_f8<RKV_APPEND_NTL>(k_new + src_of(u));
    const F8 v = load_f8<RKV_APPEND_NTL>(v_new + src_of(u));
    put(u, blk, row, k, v);
  }
}

// ---- gather -----------------------------------------------------------------
// grid = (max_blocks_per_seq * (Hkv / HPW) * ppt, num_seqs, 2 [K,V]).  A
// unit is 16 bytes of output (8 elements of a 16-bit output, 4 of an fp32
// one) and its source elements; a (block, head) tile of block_size rows is
// ppt pieces of NTH units (NTH threads a workgroup).  One workgroup moves
// piece `piece` of HPW
// consecutive heads' tiles of one block: HPW units a thread, every load
// issued before the first store.  Consecutive lanes take consecutive units
// of a tile, so loads and stores of a wave are contiguous runs: a tile's
// rows are contiguous in the pool and, for one head, in the output.  Rows
// past the context (the sequence's last block) are not stored.  DT is
// head_dim for the 32 / 64 / 128 builds (shifts), 0 for any other multiple
// of 8.  configs[1]'s gather (us per call; bf16 -> bf16, bf16 -> fp32,
// fp32 -> fp32) by heads per workgroup HPW and pieces PPW: HPW 1 212 /
// 421 / 480, 2 194 / 299 / 404, 4 198 / 332 / 433, 8 207 / 314 / 426; PPW 2
// (a whole fp32 tile) with HPW 1 303 / 401, with HPW 2 307 / 425 (all at
// 256 threads).  So 8 KiB of output per workgroup for 16-bit pools, 4 KiB
// (128 threads, below) for fp32 pools; the previous kernel, a whole block
// (8 heads, 8-16 units a thread), ran 195 / 301 / 430.
#ifndef RKV_GATHER_HPW
#define RKV_GATHER_HPW 2  // heads (tiles) per workgroup, up to num_kv_heads
#endif
#ifndef RKV_GATHER_PPW
#define RKV_GATHER_PPW 1  // pieces of each tile per workgroup
#endif
// Threads per workgroup (= units per piece): 16-bit pools, and fp32 pools.
// configs[1] (us per call; bf16 -> bf16, bf16 -> fp32, fp32 -> fp32) at
// HPW 2: 256 threads 194 / 300 / 405, 128 threads 193 / 301 / 395, 64
// threads 194 / 313 / 396; HPW 1 (one tile per workgroup): 128 threads
// 214 / 426 / 489, 64 threads (1 KiB per workgroup, the shape copy_blocks
// streams fastest in) 238 / 487 / 531 -- each workgroup waits on its table
// and length reads before its first load, which small workgroups repeat.  The workgroups of one block's head groups are
// consecutive in the grid; one head group's blocks consecutive instead (so
// that consecutive workgroups write consecutive rows) ran 197 / 313 / 416
// against 194 / 300 / 396 (HPW 1: 241 / 478 / 491, HPW 4: 203 / 335 / 440).
#ifndef RKV_GATHER_THREADS
#define RKV_GATHER_THREADS 256
#endif
#ifndef RKV_GATHER_THREADS_F32
#define RKV_GATHER_THREADS_F32 128
#endif
template <typename TIn, typename TOut, int DT, int HPW, int PPW, int NTH>
__global__ __launch_bounds__(NTH) void gather_kernel(
    TOut* __restrict__ k_out, TOut* __restrict__ v_out, const TIn* __restrict__ k_pool,
    const TIn* __restrict__ v_pool, const int32_t* __restrict__ block_tables,
    int max_blocks_per_seq, const int32_t* __restrict__ ctx_lens,
    const int64_t* __restrict__ out_offsets, int num_kv_heads, int head_dim, int block_size,
    int ppt, int64_t num_blocks, int max_ctx) {
  constexpr int EPU = 16 / sizeof(TOut);  // elements per unit
  const int D = DT ? DT : head_dim;
  const int hg = num_kv_heads / HPW;   // head groups
  const int ppb = hg * ppt;            // workgroups per block (ppt: this launch's pieces
                                       // per tile, each PPW of the tile's 256-unit pieces)
  const int j = blockIdx.x / ppb;
  const int rem = blockIdx.x - j * ppb;
  const int h0 = (rem / ppt) * HPW, piece = rem - (rem / ppt) * ppt;
  const int b = blockIdx.y;
  const bool is_v = blockIdx.z != 0;
  // the three per-sequence reads are independent: issued together
  int L = ctx_lens[b];
  const int32_t blk = block_tables[(int64_t)b * max_blocks_per_seq + j];
  int64_t seq_base = out_offsets ? out_offsets[b] : 0;
  L = L < 0 ? 0 : L;
  const int cap = max_blocks_per_seq * block_size;
  L = L > cap ? cap : L;
  int row_stride;  // output rows per head
  if (out_offsets) {
    if (seq_base < 0 || (seq_base % EPU)) return;  // 16-byte vector stores
    row_stride = L;
  } else {
    L = L > max_ctx ? max_ctx : L;
    seq_base = (int64_t)b * num_kv_heads * max_ctx * D;
    row_stride = max_ctx;
  }
  const int p0 = j * block_size;
  if (p0 >= L) return;
  if (blk < 0 || blk >= num_blocks) return;
  const int nt = (L - p0) < block_size ? (L - p0) : block_size;
  const int upr = D / EPU;          // units per row
  const int tu = block_size * upr;  // units per tile
  constexpr int LB = EPU * sizeof(TIn);  // bytes loaded per unit: 16, or 8 (bf16 -> fp32)
  using In = typename std::conditional<LB == 16, uint4, uint2>::type;
  constexpr bool NTL = RKV_GATHER_NT && sizeof(TIn) == 2;
  constexpr bool NTS = RKV_GATHER_NT && (sizeof(TOut) == 2 || RKV_GATHER_NTS_F32);
  const TIn* base = (is_v ? v_pool : k_pool) + ((int64_t)blk * num_kv_heads + h0) * block_size * D;
  const int64_t tile = (int64_t)block_size * D;  // elements per tile
  uint4 y[PPW][HPW];
#pragma unroll
  for (int q = 0; q < PPW; ++q) {
    const int u = (piece * PPW + q) * NTH + threadIdx.x;
    // loads are unconditional (a unit past the tile re-reads its last
    // unit) so each store waits for its own load only
    const int uc = u < tu ? u : tu - 1;
#pragma unroll
    for (int k = 0; k < HPW; ++k) {
      const TIn* src = base + k * tile + (int64_t)uc * EPU;
      In x;
      if constexpr (LB == 16)
        x = ld16<NTL>(src);
      else if constexpr (NTL)
        x = __builtin_bit_cast(In, __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(src)));
      else
        x = *reinterpret_cast<const In*>(src);
      if constexpr (sizeof(TIn) == 2 && sizeof(TOut) == 4)
        y[q][k] = make_uint4(x.x << 16, x.x & 0xffff0000u, x.y << 16, x.y & 0xffff0000u);
      else
        y[q][k] = x;
    }
  }
  TOut* out = (is_v ? v_out : k_out) + seq_base + ((int64_t)h0 * row_stride + p0) * D;
#pragma unroll
  for (int q = 0; q < PPW; ++q) {
    const int u = (piece * PPW + q) * NTH + threadIdx.x;
    const int rr = u / upr, c = u - rr * upr;
    if (u < tu && rr < nt) {
#pragma unroll
      for (int k = 0; k < HPW; ++k)
        store16<NTS>(out + ((int64_t)k * row_stride + rr) * D + c * EPU, y[q][k]);
    }
  }
}

// ---- copy_blocks --------------------------------------------------------------
// grid = (n_pairs * pieces, n_layers, 2 [K,V]); a piece is kCopyPiece bytes
// of a block (a bf16 block of 8 heads x 16 rows x 128 dims is 32 pieces of
// 1 KiB) and each workgroup -- one wave -- moves one piece: one 16-byte load
// and one 16-byte store per lane, one round.  Measured on this part (32 KiB
// blocks in a 4 GiB pool, GB/s moved, consecutive / random sources into
// consecutive destinations): 32 KiB per workgroup (8 loads then 8 stores a
// thread) 5.97-6.06; 4 KiB per 256-thread workgroup 6.37-6.44 / 6.41-6.44;
// 2 KiB per 128 threads 6.37-6.38 / 6.43-6.48; 1 KiB per 64 threads
// 6.66-6.69 / 6.68-6.71, as fast as a flat copy in the same shape (6.71-
// 6.75; 4 KiB per workgroup 6.51-6.53).  The smaller the work per
// workgroup, the fewer bytes the resident workgroups have in flight at once
// and the fewer DRAM rows the writes keep open.
#ifndef RKV_COPY_THREADS
#define RKV_COPY_THREADS 64
#endif
constexpr int kCopyThreads = RKV_COPY_THREADS;
constexpr int kCopyPiece = 16 * kCopyThreads;  // bytes per workgroup

__global__ __launch_bounds__(kCopyThreads) void copy_blocks_kernel(
    char* __restrict__ k_pool, char* __restrict__ v_pool, int64_t layer_stride_bytes,
    const int32_t* __restrict__ pairs, int64_t block_bytes, int pieces, int64_t num_blocks) {
  const int64_t g = blockIdx.x;
  const int64_t i = g / pieces;
  const int piece = (int)(g - i * pieces);
  const int32_t src = pairs[2 * i], dst = pairs[2 * i + 1];
  if (src < 0 || src >= num_blocks || dst < 0 || dst >= num_blocks) return;
  const int64_t off = (int64_t)piece * kCopyPiece + threadIdx.x * 16;
  if (off >= block_bytes) return;  // the last piece of a block of another size
  char* base = (blockIdx.z ? v_pool : k_pool) + blockIdx.y * layer_stride_bytes;
  const uint4 x = ld16<RKV_COPY_NTL>(base + src * block_bytes + off);
  store16<RKV_COPY_NTS>(base + dst * block_bytes + off, x);
}

// ---- 1-byte storage (int8 / fp8 e4m3, one fp32 scale per row) ---------------
// append_q: grid = (n_tokens, n_layers).  Thread u quantizes 8 elements of one
// K row and one V row (row = a KV head of the token); the D/8 threads of a row
// are consecutive lanes of one wave (D/8 in {4, 8, 16}), so the row maximum is
// a DPP group maximum.  Every thread of the workgroup runs the same number of
// rounds, so all lanes of a group take part in each reduction.
template <int D, int FMT>
__global__ __launch_bounds__(256) void append_q_kernel(
    uint8_t* __restrict__ k_pool, uint8_t* __restrict__ v_pool, float* __restrict__ k_scale,
    float* __restrict__ v_scale, int64_t pool_layer_stride, int64_t scale_layer_stride,
    const float* __restrict__ k_new, const float* __restrict__ v_new, int64_t src_layer_stride,
    int64_t src_tok_stride, int64_t src_head_stride, const int64_t* __restrict__ slot_mapping,
    int num_kv_heads, int block_size, int bs_log2, int64_t num_slots) {
  constexpr int CH = D / 8;  // threads per row
  constexpr float kTop = FMT == RKV_I8 ? 127.0f : 448.0f;
  const int t = blockIdx.x, layer = blockIdx.y;
  const int units = num_kv_heads * CH;
  const int64_t slot = slot_mapping[t];
  const bool valid = slot >= 0 && slot < num_slots;
  const int64_t blk = valid ? (bs_log2 >= 0 ? slot >> bs_log2 : slot / block_size) : 0;
  const int64_t row = slot - blk * block_size;
  for (int u0 = 0; u0 < units; u0 += blockDim.x) {
    const int u = u0 + threadIdx.x;
    const bool act = u < units;
    const int h = u / CH, c = u - h * CH;
    const int64_t src = layer * src_layer_stride + t * src_tok_stride + h * src_head_stride + c * 8;
    float kx[8], vx[8];
    if (act) {
      const F8 k = load_f8(k_new + src), v = load_f8(v_new + src);
      kx[0] = k.a.x, kx[1] = k.a.y, kx[2] = k.a.z, kx[3] = k.a.w;
      kx[4] = k.b.x, kx[5] = k.b.y, kx[6] = k.b.z, kx[7] = k.b.w;
      vx[0] = v.a.x, vx[1] = v.a.y, vx[2] = v.a.z, vx[3] = v.a.w;
      vx[4] = v.b.x, vx[5] = v.b.y, vx[6] = v.b.z, vx[7] = v.b.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) kx[e] = vx[e] = 0.0f;
    }
    float ka = 0.0f, va = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ka = fmaxf(ka, fabsf(kx[e]));
      va = fmaxf(va, fabsf(vx[e]));
    }
    ka = group_max<CH>(ka);
    va = group_max<CH>(va);
    if (!act || !valid) continue;
    const float kinv = ka > 0.0f ? kTop / ka : 0.0f, vinv = va > 0.0f ? kTop / va : 0.0f;
    uint32_t kw[2] = {0u, 0u}, vw[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t kb = FMT == RKV_I8 ? i8_quant(kx[e], kinv) : e4m3_from_f32(kx[e] * kinv);
      const uint32_t vb = FMT == RKV_I8 ? i8_quant(vx[e], vinv) : e4m3_from_f32(vx[e] * vinv);
      kw[e >> 2] |= kb << (8 * (e & 3));
      vw[e >> 2] |= vb << (8 * (e & 3));
    }
    const int64_t r = (blk * num_kv_heads + h) * block_size + row;  // row index in the layer
    const int64_t dst = layer * pool_layer_stride + r * D + c * 8;
    *reinterpret_cast<uint2*>(k_pool + dst) = make_uint2(kw[0], kw[1]);
    *reinterpret_cast<uint2*>(v_pool + dst) = make_uint2(vw[0], vw[1]);
    if (c == 0) {
      k_scale[layer * scale_layer_stride + r] = ka / kTop;
      v_scale[layer * scale_layer_stride + r] = va / kTop;
    }
  }
}

// gather_q: a thread turns one 4-byte word of a row into one float4 (byte
// value * row scale): consecutive lanes take consecutive words, so a
// wave-load reads 256 contiguous bytes and a wave-store writes 1 KiB of one
// head's contiguous output rows (writing 16 floats per lane, the stores of
// a wave were 64 bytes apart and the kernel streamed at half the rate).
// Rows past the context (the sequence's last block) are skipped.  Ordinary
// loads and nontemporal stores: 302-310 us at configs[2] (int8 / fp8)
// against 314-324 us for the other three combinations, with a whole block
// (16 words a thread) per workgroup.
#ifndef RKV_GATHER_Q_NTL
#define RKV_GATHER_Q_NTL 0
#endif
#ifndef RKV_GATHER_Q_NTS
#define RKV_GATHER_Q_NTS 1
#endif
// grid = (max_blocks_per_seq * (Hkv / HPW) * ppt, num_seqs, 2 [K,V]): one
// piece of NTH words (NTH threads) of HPW consecutive heads' (block, head) tiles per
// workgroup, HPW words (4 bytes in, 16 bytes of fp32 out each) per thread,
// one round.  configs[1]'s gather over 1-byte pools (us per call, int8 /
// fp8), 256 threads: HPW 1 493 / 505, 2 288 / 293, 4 262 / 257, 8 271 /
// 276.  One configs[2] layer of 1-byte pools into the packed layout (int8,
// us per call, one process, rotating over 32 layers) by threads x HPW:
// 128 x 4 280, 256 x 4 288-291, 256 x 8 294, 64 x 4 292, 64 x 8 299,
// 128 x 8 299-300.
#ifndef RKV_GATHER_Q_HPW
#define RKV_GATHER_Q_HPW 4
#endif
#ifndef RKV_GATHER_Q_THREADS
#define RKV_GATHER_Q_THREADS 128  // threads per workgroup = words per piece
#endif
constexpr int kGatherQThreads = RKV_GATHER_Q_THREADS;
template <int D, int FMT, int HPW>
__global__ __launch_bounds__(kGatherQThreads) void gather_q_kernel(
    float* __restrict__ k_out, float* __restrict__ v_out, const uint8_t* __restrict__ k_pool,
    const uint8_t* __restrict__ v_pool, const float* __restrict__ k_scale,
    const float* __restrict__ v_scale, const int32_t* __restrict__ block_tables,
    int max_blocks_per_seq, const int32_t* __restrict__ ctx_lens,
    const int64_t* __restrict__ out_offsets, int num_kv_heads, int block_size, int ppt,
    int64_t num_blocks, int max_ctx) {
  const int ppb = (num_kv_heads / HPW) * ppt;
  const int j = blockIdx.x / ppb;
  const int rem = blockIdx.x - j * ppb;
  const int h0 = (rem / ppt) * HPW, piece = rem - (rem / ppt) * ppt;
  const int b = blockIdx.y;
  const bool is_v = blockIdx.z != 0;
  int L = ctx_lens[b];
  const int32_t blk = block_tables[(int64_t)b * max_blocks_per_seq + j];
  int64_t seq_base = out_offsets ? out_offsets[b] : 0;
  L = L < 0 ? 0 : L;
  const int cap = max_blocks_per_seq * block_size;
  L = L > cap ? cap : L;
  int row_stride;
  if (out_offsets) {
    if (seq_base < 0 || (seq_base & 3)) return;  // 16-byte vector stores need 4-float alignment
    row_stride = L;
  } else {
    L = L > max_ctx ? max_ctx : L;
    seq_base = (int64_t)b * num_kv_heads * max_ctx * D;
    row_stride = max_ctx;
  }
  const int p0 = j * block_size;
  if (p0 >= L) return;
  if (blk < 0 || blk >= num_blocks) return;
  const int nt = (L - p0) < block_size ? (L - p0) : block_size;
  constexpr int U = D / 4;  // words per row
  const int tu = block_size * U;  // words per tile
  const int64_t row0 = ((int64_t)blk * num_kv_heads + h0) * block_size;  // first row of head h0
  const int u = piece * kGatherQThreads + threadIdx.x;
  const int uc = u < tu ? u : tu - 1;  // loads are unconditional (the tile's last word)
  const uint32_t* src = reinterpret_cast<const uint32_t*>((is_v ? v_pool : k_pool) + row0 * D);
  const float* sc = (is_v ? v_scale : k_scale) + row0;
  uint32_t w[HPW];
  float sk[HPW];
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    if constexpr (RKV_GATHER_Q_NTL) w[k] = __builtin_nontemporal_load(src + k * tu + uc);
    else w[k] = src[k * tu + uc];
    sk[k] = sc[k * block_size + uc / U];
  }
  const int rr = u / U, c = u - rr * U;
  if (u < tu && rr < nt) {
    float* dst = (is_v ? v_out : k_out) + seq_base + ((int64_t)h0 * row_stride + p0 + rr) * D + 4 * c;
#pragma unroll
    for (int k = 0; k < HPW; ++k) {
      float f[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t byte = (w[k] >> (8 * e)) & 0xffu;
        f[e] = (FMT == RKV_I8 ? (float)(int8_t)byte : f32_from_e4m3((uint8_t)byte)) * sk[k];
      }
      store16<RKV_GATHER_Q_NTS>(dst + (int64_t)k * row_stride * D,
                                make_float4(f[0], f[1], f[2], f[3]));
    }
  }
}

int check_common(int num_kv_heads, int head_dim, int block_size, int64_t num_blocks, int dtype) {
  if (num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks < 0)
    return fail(RKV_ERR_INVALID_ARG, "num_kv_heads, head_dim, block_size must be > 0");
  if (head_dim % 8) return fail(RKV_ERR_UNSUPPORTED, "head_dim must be a multiple of 8");
  if (dtype != RKV_F32 && dtype != RKV_BF16)
    return fail(RKV_ERR_INVALID_ARG, "dtype must be RKV_F32 or RKV_BF16");
  return RKV_OK;
}

}  // namespace
}  // namespace rkv

using namespace rkv;

extern "C" int rkv_append(void* k_pool, void* v_pool, int64_t pool_layer_stride,
                          const float* k_new, const float* v_new, int64_t src_layer_stride,
                          int64_t src_tok_stride, int64_t src_head_stride,
                          const int64_t* slot_mapping, int64_t n_tokens, int n_layers,
                          int num_kv_heads, int head_dim, int block_size, int64_t num_blocks,
                          int dtype, void* stream) {
  clear_error();
  if (int rc = check_common(num_kv_heads, head_dim, block_size, num_blocks, dtype)) return rc;
  if (n_tokens < 0 || n_layers < 0) return fail(RKV_ERR_INVALID_ARG, "negative n_tokens/n_layers");
  if (n_tokens == 0 || n_layers == 0) return RKV_OK;
  if (!k_pool || !v_pool || !k_new || !v_new || !slot_mapping)
    return fail(RKV_ERR_INVALID_ARG, "null pointer argument");
  if (n_tokens > 0x7fffffff || n_layers > 65535)
    return fail(RKV_ERR_INVALID_ARG, "n_tokens or n_layers too large for one launch");
  if ((src_layer_stride | src_tok_stride | src_head_stride) & 3)
    return fail(RKV_ERR_INVALID_ARG, "source strides must be multiples of 4 elements");
  if (!aligned16(k_new) || !aligned16(v_new) || !aligned16(k_pool) || !aligned16(v_pool))
    return fail(RKV_ERR_INVALID_ARG, "pointers must be 16-byte aligned");
  if (n_layers > 1 && (pool_layer_stride % 8))
    return fail(RKV_ERR_INVALID_ARG, "pool_layer_stride must be a multiple of 8 elements");
  const int units = num_kv_heads * (head_dim / 8);
  const int threads = units >= 256 ? 256 : ((units + 63) / 64) * 64;
  dim3 grid((unsigned)n_tokens, (unsigned)n_layers);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n_slots = num_blocks * block_size;
  const int bs_log2 = (block_size & (block_size - 1)) ? -1 : __builtin_ctz((unsigned)block_size);
  if (dtype == RKV_BF16)
    append_kernel<true><<<grid, threads, 0, s>>>(k_pool, v_pool, pool_layer_stride, k_new, v_new,
                                                  src_layer_stride, src_tok_stride, src_head_stride,
                                                  slot_mapping, num_kv_heads, head_dim, block_size,
                                                  bs_log2, n_slots);
  else
    append_kernel<false><<<grid, threads, 0, s>>>(k_pool, v_pool, pool_layer_stride, k_new, v_new,
                                                   src_layer_stride, src_tok_stride,
                                                   src_head_stride, slot_mapping, num_kv_heads,
                                                   head_dim, block_size, bs_log2, n_slots);
  return check_launch("rkv_append");
}

extern "C" int rkv_gather(void* k_out, void* v_out, const void* k_pool, const void* v_pool,
                          const int32_t* block_tables, int max_blocks_per_seq,
                          const int32_t* ctx_lens, const int64_t* out_offsets, int num_seqs,
                          int num_kv_heads, int head_dim, int block_size, int64_t num_blocks,
                          int max_ctx, int dtype, int out_dtype, void* stream) {
  clear_error();
  if (int rc = check_common(num_kv_heads, head_dim, block_size, num_blocks, dtype)) return rc;
  if (out_dtype != dtype && out_dtype != RKV_F32)
    return fail(RKV_ERR_INVALID_ARG, "out_dtype must equal dtype or be RKV_F32");
  if (num_seqs < 0 || max_blocks_per_seq < 0)
    return fail(RKV_ERR_INVALID_ARG, "negative num_seqs/max_blocks_per_seq");
  if (num_seqs == 0 || max_blocks_per_seq == 0) return RKV_OK;
  if (num_seqs > 65535) return fail(RKV_ERR_INVALID_ARG, "num_seqs > 65535");
  if (!k_out || !v_out || !k_pool || !v_pool || !block_tables || !ctx_lens)
    return fail(RKV_ERR_INVALID_ARG, "null pointer argument");
  if (!out_offsets && max_ctx <= 0)
    return fail(RKV_ERR_INVALID_ARG, "padded output needs max_ctx > 0");
  if (!aligned16(k_out) || !aligned16(v_out) || !aligned16(k_pool) || !aligned16(v_pool))
    return fail(RKV_ERR_INVALID_ARG, "pointers must be 16-byte aligned");
  const int epu = out_dtype == RKV_F32 ? 4 : 8;  // output elements per 16-byte unit
  const int nth = dtype == RKV_F32 ? RKV_GATHER_THREADS_F32 : RKV_GATHER_THREADS;
  const int64_t pieces = ((int64_t)block_size * (head_dim / epu) + nth - 1) / nth;
  const int ppw = pieces % RKV_GATHER_PPW == 0 ? RKV_GATHER_PPW : 1;
  const int64_t ppt = pieces / ppw;  // workgroups per tile
  // heads per workgroup: the build's choice when it divides num_kv_heads
  const int hpw = num_kv_heads % RKV_GATHER_HPW == 0 ? RKV_GATHER_HPW
                  : num_kv_heads % 4 == 0 && RKV_GATHER_HPW > 4 ? 4
                  : num_kv_heads % 2 == 0 && RKV_GATHER_HPW > 2 ? 2 : 1;
  const int64_t gx = (int64_t)max_blocks_per_seq * (num_kv_heads / hpw) * ppt;
  if (gx > INT32_MAX)
    return fail(RKV_ERR_INVALID_ARG, "max_blocks_per_seq * num_kv_heads * tile pieces exceeds 2^31 - 1");
  dim3 grid((unsigned)gx, (unsigned)num_seqs, 2);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define RKV_GATHER_HP(TI, TO, DT, H, P)                                                        \
  gather_kernel<TI, TO, DT, H, P,                                                              \
                (sizeof(TI) == 4 ? RKV_GATHER_THREADS_F32 : RKV_GATHER_THREADS)><<<grid, nth, 0, s>>>(\
      static_cast<TO*>(k_out), static_cast<TO*>(v_out), static_cast<const TI*>(k_pool),        \
      static_cast<const TI*>(v_pool), block_tables, max_blocks_per_seq, ctx_lens, out_offsets, \
      num_kv_heads, head_dim, block_size, (int)ppt, num_blocks, max_ctx)
#define RKV_GATHER_H(TI, TO, DT, H)                                    \
  do {                                                                 \
    if (ppw == RKV_GATHER_PPW) RKV_GATHER_HP(TI, TO, DT, H, RKV_GATHER_PPW); \
    else RKV_GATHER_HP(TI, TO, DT, H, 1);                              \
  } while (0)
#define RKV_GATHER_D(TI, TO, DT)                                                     \
  do {                                                                               \
    if (hpw == RKV_GATHER_HPW) RKV_GATHER_H(TI, TO, DT, RKV_GATHER_HPW);             \
    else if (hpw == 4) RKV_GATHER_H(TI, TO, DT, (RKV_GATHER_HPW > 4 ? 4 : 1));       \
    else if (hpw == 2) RKV_GATHER_H(TI, TO, DT, (RKV_GATHER_HPW > 2 ? 2 : 1));       \
    else RKV_GATHER_H(TI, TO, DT, 1);                                                \
  } while (0)
#define RKV_GATHER(TI, TO)                       \
  do {                                           \
    if (head_dim == 128) RKV_GATHER_D(TI, TO, 128); \
    else if (head_dim == 64) RKV_GATHER_D(TI, TO, 64); \
    else if (head_dim == 32) RKV_GATHER_D(TI, TO, 32); \
    else RKV_GATHER_D(TI, TO, 0);                \
  } while (0)
  if (dtype == RKV_F32)
    RKV_GATHER(float, float);
  else if (out_dtype == RKV_F32)
    RKV_GATHER(uint16_t, float);
  else
    RKV_GATHER(uint16_t, uint16_t);
#undef RKV_GATHER
#undef RKV_GATHER_D
#undef RKV_GATHER_H
#undef RKV_GATHER_HP
  return check_launch("rkv_gather");
}

namespace {
int check_q(int num_kv_heads, int head_dim, int block_size, int64_t num_blocks, int dtype) {
  if (num_kv_heads <= 0 || block_size <= 0 || num_blocks < 0)
    return fail(RKV_ERR_INVALID_ARG, "num_kv_heads and block_size must be > 0");
  if (dtype != RKV_I8 && dtype != RKV_FP8)
    return fail(RKV_ERR_INVALID_ARG, "dtype must be RKV_I8 or RKV_FP8");
  if (head_dim != 32 && head_dim != 64 && head_dim != 128)
    return fail(RKV_ERR_UNSUPPORTED, "1-byte pools: head_dim must be 32, 64 or 128");
  return RKV_OK;
}
}  // namespace

extern "C" int rkv_append_q(void* k_pool, void* v_pool, float* k_scale, float* v_scale,
                            int64_t pool_layer_stride, const float* k_new, const float* v_new,
                            int64_t src_layer_stride, int64_t src_tok_stride,
                            int64_t src_head_stride, const int64_t* slot_mapping,
                            int64_t n_tokens, int n_layers, int num_kv_heads, int head_dim,
                            int block_size, int64_t num_blocks, int dtype, void* stream) {
  clear_error();
  if (int rc = check_q(num_kv_heads, head_dim, block_size, num_blocks, dtype)) return rc;
  if (n_tokens < 0 || n_layers < 0) return fail(RKV_ERR_INVALID_ARG, "negative n_tokens/n_layers");
  if (n_tokens == 0 || n_layers == 0) return RKV_OK;
  if (!k_pool || !v_pool || !k_scale || !v_scale || !k_new || !v_new || !slot_mapping)
    return fail(RKV_ERR_INVALID_ARG, "null pointer argument");
  if (n_tokens > 0x7fffffff || n_layers > 65535)
    return fail(RKV_ERR_INVALID_ARG, "n_tokens or n_layers too large for one launch");
  if ((src_layer_stride | src_tok_stride | src_head_stride) & 3)
    return fail(RKV_ERR_INVALID_ARG, "source strides must be multiples of 4 elements");
  if (!aligned16(k_new) || !aligned16(v_new) || !aligned16(k_pool) || !aligned16(v_pool))
    return fail(RKV_ERR_INVALID_ARG, "pointers must be 16-byte aligned");
  if (n_layers > 1 && (pool_layer_stride % 16))
    return fail(RKV_ERR_INVALID_ARG, "pool_layer_stride must be a multiple of 16 bytes");
  const int units = num_kv_heads * (head_dim / 8);
  const int threads = units >= 256 ? 256 : ((units + 63) / 64) * 64;
  const dim3 grid((unsigned)n_tokens, (unsigned)n_layers);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n_slots = num_blocks * block_size;
  const int bs_log2 = (block_size & (block_size - 1)) ? -1 : __builtin_ctz((unsigned)block_size);
  // scales: one per row; a layer of the scale pool holds num_blocks * Hkv * block_size
  const int64_t scale_ls = n_layers > 1 ? pool_layer_stride / head_dim : 0;
#define RKV_APPEND_Q(D, F)                                                                      \
  append_q_kernel<D, F><<<grid, threads, 0, s>>>(                                               \
      static_cast<uint8_t*>(k_pool), static_cast<uint8_t*>(v_pool), k_scale, v_scale,           \
      pool_layer_stride, scale_ls, k_new, v_new, src_layer_stride, src_tok_stride,              \
      src_head_stride, slot_mapping, num_kv_heads, block_size, bs_log2, n_slots)
  if (dtype == RKV_I8) {
    if (head_dim == 32) RKV_APPEND_Q(32, RKV_I8);
    else if (head_dim == 64) RKV_APPEND_Q(64, RKV_I8);
    else RKV_APPEND_Q(128, RKV_I8);
  } else {
    if (head_dim == 32) RKV_APPEND_Q(32, RKV_FP8);
    else if (head_dim == 64) RKV_APPEND_Q(64, RKV_FP8);
    else RKV_APPEND_Q(128, RKV_FP8);
  }
#undef RKV_APPEND_Q
  return check_launch("rkv_append_q");
}

extern "C" int rkv_gather_q(float* k_out, float* v_out, const void* k_pool, const void* v_pool,
                            const float* k_scale, const float* v_scale,
                            const int32_t* block_tables, int max_blocks_per_seq,
                            const int32_t* ctx_lens, const int64_t* out_offsets, int num_seqs,
                            int num_kv_heads, int head_dim, int block_size, int64_t num_blocks,
                            int max_ctx, int dtype, void* stream) {
  clear_error();
  if (int rc = check_q(num_kv_heads, head_dim, block_size, num_blocks, dtype)) return rc;
  if (num_seqs < 0 || max_blocks_per_seq < 0)
    return fail(RKV_ERR_INVALID_ARG, "negative num_seqs/max_blocks_per_seq");
  if (num_seqs == 0 || max_blocks_per_seq == 0) return RKV_OK;
  if (num_seqs > 65535) return fail(RKV_ERR_INVALID_ARG, "num_seqs > 65535");
  if (!k_out || !v_out || !k_pool || !v_pool || !k_scale || !v_scale || !block_tables ||
      !ctx_lens)
    return fail(RKV_ERR_INVALID_ARG, "null pointer argument");
  if (!out_offsets && max_ctx <= 0)
    return fail(RKV_ERR_INVALID_ARG, "padded output needs max_ctx > 0");
  if (!aligned16(k_out) || !aligned16(v_out) || !aligned16(k_pool) || !aligned16(v_pool))
    return fail(RKV_ERR_INVALID_ARG, "pointers must be 16-byte aligned");
  const int64_t ppt =
      ((int64_t)block_size * (head_dim / 4) + kGatherQThreads - 1) / kGatherQThreads;
  const int hpw = num_kv_heads % RKV_GATHER_Q_HPW == 0 ? RKV_GATHER_Q_HPW
                  : num_kv_heads % 4 == 0 && RKV_GATHER_Q_HPW > 4 ? 4
                  : num_kv_heads % 2 == 0 && RKV_GATHER_Q_HPW > 2 ? 2 : 1;
  const int64_t gx = (int64_t)max_blocks_per_seq * (num_kv_heads / hpw) * ppt;
  if (gx > INT32_MAX)
    return fail(RKV_ERR_INVALID_ARG, "max_blocks_per_seq * num_kv_heads * tile pieces exceeds 2^31 - 1");
  const dim3 grid((unsigned)gx, (unsigned)num_seqs, 2);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define RKV_GATHER_QH(D, F, H)                                                                  \
  gather_q_kernel<D, F, H><<<grid, kGatherQThreads, 0, s>>>(                                    \
      k_out, v_out, static_cast<const uint8_t*>(k_pool), static_cast<const uint8_t*>(v_pool),   \
      k_scale, v_scale, block_tables, max_blocks_per_seq, ctx_lens, out_offsets, num_kv_heads,  \
      block_size, (int)ppt, num_blocks, max_ctx)
#define RKV_GATHER_Q(D, F)                                                   \
  do {                                                                       \
    if (hpw == RKV_GATHER_Q_HPW) RKV_GATHER_QH(D, F, RKV_GATHER_Q_HPW);      \
    else if (hpw == 4) RKV_GATHER_QH(D, F, (RKV_GATHER_Q_HPW > 4 ? 4 : 1));  \
    else if (hpw == 2) RKV_GATHER_QH(D, F, (RKV_GATHER_Q_HPW > 2 ? 2 : 1));  \
    else RKV_GATHER_QH(D, F, 1);                                             \
  } while (0)
  if (dtype == RKV_I8) {
    if (head_dim == 32) RKV_GATHER_Q(32, RKV_I8);
    else if (head_dim == 64) RKV_GATHER_Q(64, RKV_I8);
    else RKV_GATHER_Q(128, RKV_I8);
  } else {
    if (head_dim == 32) RKV_GATHER_Q(32, RKV_FP8);
    else if (head_dim == 64) RKV_GATHER_Q(64, RKV_FP8);
    else RKV_GATHER_Q(128, RKV_FP8);
  }
#undef RKV_GATHER_Q
#undef RKV_GATHER_QH
  return check_launch("rkv_gather_q");
}

extern "C" int rkv_copy_blocks(void* k_pool, void* v_pool, int64_t layer_stride_bytes,
                               int n_layers, const int32_t* pairs, int n_pairs,
                               int64_t block_bytes, int64_t num_blocks, void* stream) {
  clear_error();
  if (n_pairs < 0 || n_layers < 0) return fail(RKV_ERR_INVALID_ARG, "negative n_pairs/n_layers");
  if (n_pairs == 0 || n_layers == 0) return RKV_OK;
  if (!k_pool || !v_pool || !pairs) return fail(RKV_ERR_INVALID_ARG, "null pointer argument");
  if (block_bytes <= 0 || (block_bytes & 15))
    return fail(RKV_ERR_INVALID_ARG, "block_bytes must be a positive multiple of 16");
  if (n_layers > 65535) return fail(RKV_ERR_INVALID_ARG, "n_layers > 65535");
  if (n_layers > 1 && (layer_stride_bytes & 15))
    return fail(RKV_ERR_INVALID_ARG, "layer_stride_bytes must be a multiple of 16");
  if (!aligned16(k_pool) || !aligned16(v_pool))
    return fail(RKV_ERR_INVALID_ARG, "pools must be 16-byte aligned");
  const int64_t pieces = (block_bytes + kCopyPiece - 1) / kCopyPiece;
  if ((int64_t)n_pairs * pieces > INT32_MAX)
    return fail(RKV_ERR_INVALID_ARG, "n_pairs * ceil(block_bytes / " + std::to_string(kCopyPiece) +
                                         ") exceeds 2^31 - 1");
  dim3 grid((unsigned)(n_pairs * pieces), (unsigned)n_layers, 2);
  copy_blocks_kernel<<<grid, kCopyThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<char*>(k_pool), static_cast<char*>(v_pool), layer_stride_bytes, pairs,
      block_bytes, (int)pieces, num_blocks);
  return check_launch("rkv_copy_blocks");
}
