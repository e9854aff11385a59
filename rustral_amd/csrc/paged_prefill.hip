// paged_prefill.hip -- causal prefill attention over the paged KV pool, for
// gfx950 (CDNA4, wave64): many new query tokens per sequence attend to the
// cached tokens and to each other (causal), reading K/V through the block
// table.  The new tokens' K/V are appended to the pool first (rkv_append).
//
// One workgroup per (tile of 16 * QS query tokens, KV head, sequence),
// (G / HW) * QS waves: wave (g, t) serves the HW query heads kh * G + HW g ..
// for the t-th 16-token sub-tile, so each K/V byte staged in LDS serves G
// heads x QS sub-tiles, and each K/V fragment a wave reads from LDS feeds the
// MFMAs of HW heads (two independent dependency chains per wave for HW = 2).
// The workgroup walks the 16-token blocks, KB per iteration, from position 0
// to the tile's last query position:
//   * stage: the KB blocks' K and V tiles go through registers into LDS,
//     row-major with padded rows, double buffered; the loads run two
//     iterations ahead of the compute.
//     A wave skips the arithmetic of key blocks that lie entirely after its
//     last query (causal).
//   * S^T = K Q^T on v_mfma_f32_16x16x32_bf16: A = K rows from LDS, B = Q^T
//     (queries of the 16 tokens, split hi + lo bf16 so the scores carry ~16
//     significant bits of q).  Result: lane l holds S^T[key 4(l/16)+r][row
//     l%16] -- every value a lane holds belongs to query row l % 16.
//   * causal mask (key position > query position -> excluded), then an
//     online softmax per row (reductions over the row's four lanes by
//     permlane swaps): running max m and sum l, the accumulator
//     rescaled by 2^(m_old - m_new).  Scores carry scale * log2(e) (exp2).
//   * O^T += V^T P^T on v_mfma_f32_16x16x32_bf16 over two key blocks at a
//     time (16x16x16 for an odd KB): A = V^T, read from the row-major V tile
//     by ds_read_b64_tr_b16 (a transposing LDS read), B = P^T, which is
//     exactly the S^T layout above (no cross-lane moves); P is split hi + lo
//     like q.  Result: lane l holds O^T[dim 16c + 4(l/16)+r][row l%16].
// fp32 pools split K and V into hi + lo bf16 as well (three products each).
// MFMA lane layouts (gfx950): 16x16x32: A[l%16][8(l/16)+e], B[8(l/16)+e][l%16];
// 16x16x16: A[l%16][4(l/16)+e], B[4(l/16)+e][l%16]; both D[4(l/16)+r][l%16].
#include "common.hpp"

#include <cmath>
#include <mutex>
#include <type_traits>

namespace rkv {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) short bf16x4_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kBS = 16;  // tokens per block = keys per staged block

// max(a, b) as v_med3_f32(a, b, +inf): one instruction, without the
// quieting copies fmaxf gets in IEEE mode (the values here are never NaN).
__device__ __forceinline__ float max2(float a, float b) {
  return __builtin_amdgcn_fmed3f(a, b, INFINITY);
}

// x combined with x of lane l ^ 16, then of lane l ^ 32, through
// v_permlane16_swap / v_permlane32_swap (VALU, no LDS round trip).  Called with
// the same value twice, a swap returns the pair (x[l], x[l^16]) in some order,
// so the sum or maximum equals that of a __shfl_xor exchange bit for bit.
__device__ __forceinline__ float xor48_max(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = max2(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor48_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// hi = bf16(x), lo = bf16(x - hi), packed in pairs (element 2i in the low half).
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = cvt_bf16x2(a, b);
  lo = cvt_bf16x2(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xffff0000u));
}

template <typename T, int D, int G, int HW, int QS, int KB, bool PFN>
__global__ __launch_bounds__(64 * (G / HW) * QS) __attribute__((amdgpu_waves_per_eu(2))) void prefill_kernel(
    float* __restrict__ out, const float* __restrict__ q, const void* __restrict__ k_pool_,
    const void* __restrict__ v_pool_, const int32_t* __restrict__ block_tables,
    int max_blocks_per_seq, const int32_t* __restrict__ q_start,
    const int32_t* __restrict__ ctx_lens, int num_kv_heads, int64_t num_blocks, int max_q_len,
    float q_scale, int heavy_first, int pf_stride, int pf_first) {
  constexpr bool F32 = sizeof(T) == 4;
  static_assert(G % HW == 0, "heads per wave must divide the group");
  constexpr int NT = 64 * (G / HW) * QS;
  constexpr int QT = 16 * QS;              // query tokens per workgroup
  constexpr int NS = F32 ? 2 : 1;          // bf16 slices per staged element (hi, lo)
  constexpr int KP = D + 8;                // padded K row in LDS (bf16 elements)
  constexpr int VKP = D + 16;              // padded V row: the 4 rows of one transposing
                                           // read (8 bytes x 16 lanes) hit distinct banks
  constexpr int CE = 16 / sizeof(T);       // elements per 16-byte chunk
  constexpr int CPR = D / CE;              // chunks per token row
  constexpr int CH = kBS * CPR;            // chunks per (block, head) tile
  constexpr int PT = (KB * CH + NT - 1) / NT;  // chunks per thread and iteration
  constexpr int NC = D / 32;               // QK^T MFMAs per key block (per slice)
  constexpr int NO = D / 16;               // PV MFMAs per key block (per slice)
  // The output rows go out through LDS: each wave writes one head's 16 rows
  // (MFMA layout) into wave-private rows of D floats padded by 16 bytes
  // (the 16 rows of one write then fall on distinct banks) and stores them
  // back whole, 512 contiguous bytes per half-wave, where the MFMA layout
  // stored 16 rows x 64 bytes per instruction.  The rows sit after the K/V
  // staging buffers, so no workgroup barrier separates them from the loop.
  // configs[4] admissions (us per call, one box, one process): 30.5 with
  // stores from the MFMA layout, 28.0 through the rows; q staged the same
  // way as well 30.0 (its LDS round trip costs more than the contiguous
  // loads save), both heads' rows at once behind a workgroup barrier 28.7.
  // Builds of one head per wave hold two workgroups per CU, which the rows'
  // LDS would halve: they store from the MFMA layout.
  constexpr bool STAGE_OUT = HW > 1;
  constexpr int NW = NT / 64;                         // waves
  constexpr int RWO = D + 4;                          // padded output row (floats)
  constexpr int KB_BYTES = 2 * NS * KB * kBS * KP * 2;
  constexpr int KV_BYTES = KB_BYTES + 2 * NS * KB * kBS * VKP * 2;
  constexpr int LDS_BYTES = KV_BYTES + (STAGE_OUT ? NW * 16 * RWO * 4 : 0);
  static_assert(KB_BYTES % 16 == 0 && KV_BYTES % 16 == 0, "16-byte aligned regions");
  __shared__ __align__(16) uint8_t s_raw[LDS_BYTES];
  auto s_k = reinterpret_cast<uint16_t (*)[NS][KB * kBS * KP]>(s_raw);
  auto s_v = reinterpret_cast<uint16_t (*)[NS][KB * kBS * VKP]>(s_raw + KB_BYTES);

  const T* __restrict__ k_pool = static_cast<const T*>(k_pool_);
  const T* __restrict__ v_pool = static_cast<const T*>(v_pool_);
  // Grid order.  heavy_first: x = KV head + num_kv_heads * sequence, y = the
  // query tiles from the last (the most keys) down, so the longest tiles are
  // dispatched first and the tiles of one (KV head, sequence) share an XCD's
  // L2 when num_kv_heads * num_seqs is a multiple of 8 (workgroups go to the
  // XCDs round robin).  Otherwise x = query tile, y = KV head, z = sequence.
  const int qt = heavy_first ? (int)(gridDim.y - 1 - blockIdx.y) : (int)blockIdx.x;
  const int kh = heavy_first ? (int)(blockIdx.x % num_kv_heads) : (int)blockIdx.y;
  const int b = heavy_first ? (int)(blockIdx.x / num_kv_heads) : (int)blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = w % (G / HW), rt = w / (G / HW);  // head set within the group, row sub-tile
  const int num_q_heads = num_kv_heads * G, h0 = kh * G + g * HW;  // the wave's first head

  const int s0 = q_start[b];
  const int n = q_start[b + 1] - s0;
  const int nr = n < max_q_len ? n : max_q_len;  // rows computed (the first nr new tokens)
  const int q0 = qt * QT;
  if (q0 >= nr) return;
  const int cap = max_blocks_per_seq * kBS;
  const int pos0 = ctx_lens[b] - n;  // position of the first new token (may be < 0)
  int last = pos0 + (q0 + QT < nr ? q0 + QT : nr) - 1;  // the workgroup's last query position
  last = last < cap - 1 ? last : cap - 1;
  const int nblk = last < 0 ? 0 : last / kBS + 1;
  const int nit = (nblk + KB - 1) / KB;

  const int r16 = lane & 15, grp = lane >> 4;
  const int qr0 = q0 + 16 * rt;      // this wave's first query row
  const bool active = qr0 < nr;      // wave-uniform: the sub-tile holds a query
  const int qi = qr0 + r16;          // this lane's query row
  const bool row_ok = qi < nr;
  const int qpos = pos0 + qi;
  const int wlast = pos0 + (qr0 + 16 < nr ? qr0 + 16 : nr) - 1;  // this wave's last query position

  const int32_t* __restrict__ tab = block_tables + (int64_t)b * max_blocks_per_seq;
  // Block ids are wave-uniform loads (scalar memory, counted apart from the
  // K/V vector loads), read one iteration before the fetch that uses them,
  // so the fetch neither waits on the table nor on earlier K/V loads.
  auto load_ids = [&](int it, int32_t (&id)[KB]) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int j = it * KB + kb;
      id[kb] = j < nblk ? tab[j] : -1;
    }
  };
  // Two register sets: the loads of iteration it + 2 are issued while
  // iteration it is computed (one workgroup fills a CU, so its own loads
  // have to be in flight early).
  u32x4_t kr0[PT], vr0[PT], kr1[PT], vr1[PT];
  // Issues the K/V loads of the KB blocks with ids id into registers;
  // returns a bit per block whose id is valid.
  auto fetch = [&](const int32_t (&id)[KB], u32x4_t (&kr)[PT], u32x4_t (&vr)[PT])
                   __attribute__((always_inline)) {
    uint32_t okm = 0;
    int64_t base[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int32_t blk = id[kb];
      const bool ok = blk >= 0 && blk < num_blocks;
      okm |= ok ? 1u << kb : 0u;
      base[kb] = ((int64_t)(ok ? blk : 0) * num_kv_heads + kh) * kBS * D;
    }
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const int ci = tid + i * NT;
      if ((KB * CH) % NT == 0 || ci < KB * CH) {
        const int kb = ci / CH, cc = ci % CH;
        int64_t bb = base[0];  // base[kb] by selects (kb is not a compile-time index)
#pragma unroll
        for (int x = 1; x < KB; ++x) bb = kb == x ? base[x] : bb;
        kr[i] = *reinterpret_cast<const u32x4_t*>(k_pool + bb + cc * CE);
        vr[i] = *reinterpret_cast<const u32x4_t*>(v_pool + bb + cc * CE);
      }
    }
    return okm;
  };
  // Writes the registers into LDS buffer buf (K and V row-major).
  auto stage = [&](int buf, const u32x4_t (&kr)[PT], const u32x4_t (&vr)[PT])
                   __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const int ci = tid + i * NT;
      if ((KB * CH) % NT == 0 || ci < KB * CH) {
        const int kb = ci / CH, cc = ci % CH;
        const int key = cc / CPR, col = (cc % CPR) * CE;
        uint16_t* kd = &s_k[buf][0][(kb * kBS + key) * KP + col];
        uint16_t* vd = &s_v[buf][0][(kb * kBS + key) * VKP + col];
        if constexpr (!F32) {
          *reinterpret_cast<u32x4_t*>(kd) = kr[i];
          *reinterpret_cast<u32x4_t*>(vd) = vr[i];
        } else {
          constexpr int KS = KB * kBS * KP, VS = KB * kBS * VKP;  // slice strides
          const float kf[4] = {__uint_as_float(kr[i].x), __uint_as_float(kr[i].y),
                               __uint_as_float(kr[i].z), __uint_as_float(kr[i].w)};
          const float vf[4] = {__uint_as_float(vr[i].x), __uint_as_float(vr[i].y),
                               __uint_as_float(vr[i].z), __uint_as_float(vr[i].w)};
          uint2 kh2, kl2;
          split2(kf[0], kf[1], kh2.x, kl2.x);
          split2(kf[2], kf[3], kh2.y, kl2.y);
          *reinterpret_cast<uint2*>(kd) = kh2;
          *reinterpret_cast<uint2*>(kd + KS) = kl2;
          uint2 vh2, vl2;
          split2(vf[0], vf[1], vh2.x, vl2.x);
          split2(vf[2], vf[3], vh2.y, vl2.y);
          *reinterpret_cast<uint2*>(vd) = vh2;
          *reinterpret_cast<uint2*>(vd + VS) = vl2;
        }
      }
    }
  };

  // This wave's q rows, loaded first: their conversion then waits for them
  // alone, not for the K/V loads queued behind.
  float4 qraw[HW][NC][2];
#pragma unroll
  for (int hh = 0; hh < HW; ++hh) {
    const float* qp =
        q + ((int64_t)(s0 + (row_ok ? qi : q0)) * num_q_heads + h0 + hh) * D + 8 * grp;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      qraw[hh][c][0] = reinterpret_cast<const float4*>(qp + 32 * c)[0];
      qraw[hh][c][1] = reinterpret_cast<const float4*>(qp + 32 * c)[1];
    }
  }
  // every q load is issued before the K/V fetches below
  __builtin_amdgcn_sched_barrier(0);

  int32_t ids[KB];
  load_ids(0, ids);
  // Every fetch is issued, also past the last iteration (ids -1: block 0's
  // tile is read and never used), so each body issues the same loads and the
  // compiler's load counters wait for exactly the set being staged.
  uint32_t ok0 = fetch(ids, kr0, vr0);
  load_ids(1, ids);
  uint32_t ok1 = fetch(ids, kr1, vr1);
  load_ids(2, ids);  // for the first fetch inside the loop
  __builtin_amdgcn_sched_barrier(0);

  // B operand of S^T = K Q^T: Q[row r16][32c + 8 grp .. + 8] * q_scale, hi
  // and lo (scores come out already scaled by scale * log2 e), converted
  // from the raw rows loaded before the first K/V fetch.
  uint4 qhi[HW][NC], qlo[HW][NC];
#pragma unroll
  for (int hh = 0; hh < HW; ++hh)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float4 x = qraw[hh][c][0], y = qraw[hh][c][1];
      if (!row_ok) x = y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      x.x *= q_scale; x.y *= q_scale; x.z *= q_scale; x.w *= q_scale;
      y.x *= q_scale; y.y *= q_scale; y.z *= q_scale; y.w *= q_scale;
      split2(x.x, x.y, qhi[hh][c].x, qlo[hh][c].x);
      split2(x.z, x.w, qhi[hh][c].y, qlo[hh][c].y);
      split2(y.x, y.y, qhi[hh][c].z, qlo[hh][c].z);
      split2(y.z, y.w, qhi[hh][c].w, qlo[hh][c].w);
    }

  f32x4_t o[HW][NO];
  float m[HW], l[HW];
#pragma unroll
  for (int hh = 0; hh < HW; ++hh) {
#pragma unroll
    for (int c = 0; c < NO; ++c) o[hh][c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    m[hh] = -INFINITY;
    l[hh] = 0.0f;
  }

  // PFN: workgroups from pf_first on touch the q rows of the workgroup
  // pf_stride places later in dispatch order (one that starts when a slot of
  // the first round frees up, on the same XCD when pf_stride is a multiple
  // of 8), one 4-byte load per 64-byte line, while they compute and HBM has
  // little else to do: that workgroup then finds them in the caches instead
  // of queueing behind the first round's output stores.  Issued after this
  // wave's q and first K/V loads, so waits for those are not held up; the
  // values are consumed (by an empty asm) only at the end of the kernel.
  constexpr int LPR = G * D * 4 / 64;  // 64-byte lines of one (token, KV head) q row
  constexpr int PF = PFN ? (QT * LPR + NT - 1) / NT : 1;
  float pfv[PF];
  if constexpr (PFN) {
    const int64_t self = (int64_t)blockIdx.x + (int64_t)gridDim.x * blockIdx.y;
    const int64_t j = self + pf_stride;
    const bool pf_on =
        heavy_first && pf_stride > 0 && self >= pf_first && j < (int64_t)gridDim.x * gridDim.y;
    const int jx = pf_on ? (int)(j % gridDim.x) : 0, jy = pf_on ? (int)(j / gridDim.x) : 0;
    const int jqt = (int)gridDim.y - 1 - jy, jkh = jx % num_kv_heads, jb = jx / num_kv_heads;
    const int js0 = pf_on ? q_start[jb] : 0;
    const int jn = pf_on ? q_start[jb + 1] - js0 : 0;
    const int jnr = jn < max_q_len ? jn : max_q_len;
    const int jq0 = jqt * QT;
    const int jrows = jnr - jq0 < QT ? jnr - jq0 : QT;  // <= 0: nothing to touch
#pragma unroll
    for (int i = 0; i < PF; ++i) pfv[i] = 0.0f;
    if (pf_on && jrows > 0) {  // workgroup-uniform
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int u = tid + i * NT, row = u / LPR, line = u % LPR;
        const bool on = u < QT * LPR && row < jrows;
        // off: this wave's own first q line (already loaded) is read again
        const int64_t off =
            on ? ((int64_t)(js0 + jq0 + row) * num_q_heads + jkh * G) * D + 16 * line
               : ((int64_t)(s0 + (row_ok ? qi : q0)) * num_q_heads + h0) * D;
        pfv[i] = q[off];
      }
    }
  }

  // Iteration it on LDS buffer buf (okm: valid blocks of the iteration).
  // MASKED: some key of the iteration is invalid or after some query of the
  // wave (the choice is made before any MFMA, so the MFMA results are read
  // in the block that computes them).
  auto compute = [&](auto masked, int it, int buf, uint32_t okm) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked)::value;
    const int kfirst = it * KB * kBS;

    // ---- S^T - m = K Q^T - m for the KB * 16 keys, per head ----
    // The accumulators start at -mref (the row's reference maximum, 0 before
    // the row has seen a key), so the scores come out of the matrix cores
    // already relative to it: no subtraction before the exponentials.
    float mref[HW];
#pragma unroll
    for (int hh = 0; hh < HW; ++hh) mref[hh] = m[hh] == -INFINITY ? 0.0f : m[hh];
    float s[HW][KB][4];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      f32x4_t st[HW];
#pragma unroll
      for (int hh = 0; hh < HW; ++hh) st[hh] = f32x4_t{-mref[hh], -mref[hh], -mref[hh], -mref[hh]};
      const uint16_t* kr0 = &s_k[buf][0][(kb * kBS + r16) * KP + 8 * grp];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint4 ka = *reinterpret_cast<const uint4*>(kr0 + 32 * c);
#pragma unroll
        for (int hh = 0; hh < HW; ++hh)
          st[hh] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, ka), __builtin_bit_cast(bf16x8_t, qhi[hh][c]), st[hh],
              0, 0, 0);
#pragma unroll
        for (int hh = 0; hh < HW; ++hh)
          st[hh] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, ka), __builtin_bit_cast(bf16x8_t, qlo[hh][c]), st[hh],
              0, 0, 0);
        if constexpr (F32) {
          const uint4 kl =
              *reinterpret_cast<const uint4*>(kr0 + KB * kBS * KP + 32 * c);
#pragma unroll
          for (int hh = 0; hh < HW; ++hh)
            st[hh] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8_t, kl), __builtin_bit_cast(bf16x8_t, qhi[hh][c]),
                st[hh], 0, 0, 0);
        }
      }
      if constexpr (MASKED) {
        // causal mask: key 4 grp + r of the block is kept when r <= lim
        const int kp0 = kfirst + kb * kBS + 4 * grp;
        const int lim = ((okm >> kb) & 1u) && row_ok ? qpos - kp0 : -1;
#pragma unroll
        for (int hh = 0; hh < HW; ++hh)
#pragma unroll
          for (int r = 0; r < 4; ++r) s[hh][kb][r] = r <= lim ? st[hh][r] : -INFINITY;
      } else {
#pragma unroll
        for (int hh = 0; hh < HW; ++hh)
#pragma unroll
          for (int r = 0; r < 4; ++r) s[hh][kb][r] = st[hh][r];
      }
    }
    // ---- online softmax of row r16, per head ----
    // The reference maximum m moves only when a row's maximum exceeds it by
    // more than kSlack (log2 units, a factor 2^8): exponentials stay <= 2^8,
    // exact in fp32 and split hi + lo as before, and the rare rescale of the
    // accumulators is one wave-uniform branch for all heads of the wave.
    // Whether some row needs it is decided from each lane's own keys (a
    // row's maximum exceeds m + kSlack iff one of its lanes' does), so the
    // cross-lane maximum is only taken inside the branch.
    constexpr float kSlack = 8.0f;
    float lm[HW];
    bool up = false;
#pragma unroll
    for (int hh = 0; hh < HW; ++hh) {
      float mb = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
        mb = max2(mb, max2(max2(s[hh][kb][0], s[hh][kb][1]), max2(s[hh][kb][2], s[hh][kb][3])));
      lm[hh] = mb;  // relative to mref
      // before the row's first key (m = -inf) any key moves m
      up = up || mb > (m[hh] == -INFINITY ? -INFINITY : kSlack);
    }
    if (__builtin_amdgcn_ballot_w64(up) != 0) {
#pragma unroll
      for (int hh = 0; hh < HW; ++hh) {
        const float mx = xor48_max(lm[hh]);  // the row's maximum, relative to mref
        const float mn = max2(m[hh], mx == -INFINITY ? -INFINITY : mx + mref[hh]);
        const float mref_new = mn == -INFINITY ? 0.0f : mn;
        // rows without any key so far (m = -inf) get alpha = 0 on o = l = 0
        const float alpha = __builtin_amdgcn_exp2f(m[hh] - mref_new);
        l[hh] *= alpha;
#pragma unroll
        for (int c = 0; c < NO; ++c)
#pragma unroll
          for (int r = 0; r < 4; ++r) o[hh][c][r] *= alpha;
        m[hh] = mn;
        const float d = mref_new - mref[hh];  // the scores move to the new reference
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) s[hh][kb][r] -= d;
      }
    }
#pragma unroll
    for (int hh = 0; hh < HW; ++hh) {
      float ls = 0.0f;
      // v_exp_f32 directly: exp2(-inf) = 0, results below 2^-126 do not matter
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          s[hh][kb][r] = __builtin_amdgcn_exp2f(s[hh][kb][r]);
          ls += s[hh][kb][r];
        }
      l[hh] += ls;  // this lane's keys of the row; the row's lanes are summed at the end
    }

    // ---- O^T += V^T P^T ----
    if constexpr (KB % 2 == 0) {
      // Two key blocks per v_mfma_f32_16x16x32_bf16: k-slot 8 grp + e holds
      // key 4 grp + e of the first block (e < 4) or of the second (e >= 4),
      // which is where this lane's P^T values are; V^T is read with the same
      // key order (one transposing read per block).
#pragma unroll
      for (int kb = 0; kb < KB; kb += 2) {
        uint4 ph[HW], pl[HW];
#pragma unroll
        for (int hh = 0; hh < HW; ++hh) {
          split2(s[hh][kb][0], s[hh][kb][1], ph[hh].x, pl[hh].x);
          split2(s[hh][kb][2], s[hh][kb][3], ph[hh].y, pl[hh].y);
          split2(s[hh][kb + 1][0], s[hh][kb + 1][1], ph[hh].z, pl[hh].z);
          split2(s[hh][kb + 1][2], s[hh][kb + 1][3], ph[hh].w, pl[hh].w);
        }
        // this lane's transposing-read address: key 4 grp + (r16 >> 2),
        // dims 16 c + 4 (r16 & 3) .. + 3
        const uint16_t* va0 = &s_v[buf][0][(kb * kBS + 4 * grp + (r16 >> 2)) * VKP + 4 * (r16 & 3)];
        const uint16_t* va1 = va0 + kBS * VKP;  // the next block
#pragma unroll
        for (int c = 0; c < NO; ++c) {
          const uint2 a0 = lds_read_tr16(va0 + 16 * c);
          const uint2 a1 = lds_read_tr16(va1 + 16 * c);
          const uint4 va = make_uint4(a0.x, a0.y, a1.x, a1.y);
#pragma unroll
          for (int hh = 0; hh < HW; ++hh)
            o[hh][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8_t, va), __builtin_bit_cast(bf16x8_t, ph[hh]), o[hh][c],
                0, 0, 0);
#pragma unroll
          for (int hh = 0; hh < HW; ++hh)
            o[hh][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8_t, va), __builtin_bit_cast(bf16x8_t, pl[hh]), o[hh][c],
                0, 0, 0);
          if constexpr (F32) {
            const uint2 l0 = lds_read_tr16(va0 + KB * kBS * VKP + 16 * c);
            const uint2 l1 = lds_read_tr16(va1 + KB * kBS * VKP + 16 * c);
            const uint4 vl = make_uint4(l0.x, l0.y, l1.x, l1.y);
#pragma unroll
            for (int hh = 0; hh < HW; ++hh)
              o[hh][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  __builtin_bit_cast(bf16x8_t, vl), __builtin_bit_cast(bf16x8_t, ph[hh]),
                  o[hh][c], 0, 0, 0);
          }
        }
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        uint2 ph[HW], pl[HW];
#pragma unroll
        for (int hh = 0; hh < HW; ++hh) {
          split2(s[hh][kb][0], s[hh][kb][1], ph[hh].x, pl[hh].x);
          split2(s[hh][kb][2], s[hh][kb][3], ph[hh].y, pl[hh].y);
        }
        const uint16_t* vr0 = &s_v[buf][0][(kb * kBS + 4 * grp + (r16 >> 2)) * VKP + 4 * (r16 & 3)];
#pragma unroll
        for (int c = 0; c < NO; ++c) {
          const uint2 va = lds_read_tr16(vr0 + 16 * c);
#pragma unroll
          for (int hh = 0; hh < HW; ++hh) {
            o[hh][c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                __builtin_bit_cast(bf16x4_t, va), __builtin_bit_cast(bf16x4_t, ph[hh]), o[hh][c],
                0, 0, 0);
            o[hh][c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                __builtin_bit_cast(bf16x4_t, va), __builtin_bit_cast(bf16x4_t, pl[hh]), o[hh][c],
                0, 0, 0);
          }
          if constexpr (F32) {
            const uint2 vl = lds_read_tr16(vr0 + KB * kBS * VKP + 16 * c);
#pragma unroll
            for (int hh = 0; hh < HW; ++hh)
              o[hh][c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                  __builtin_bit_cast(bf16x4_t, vl), __builtin_bit_cast(bf16x4_t, ph[hh]),
                  o[hh][c], 0, 0, 0);
          }
        }
      }
    }
    };
  // Iteration it on buffer buf: skipped when no row of the wave attends to
  // any of its keys.
  auto step = [&](auto masked, int it, int buf, uint32_t okm) __attribute__((always_inline)) {
    if (active && it * KB * kBS <= wlast) compute(masked, it, buf, okm);
  };
  // Iterations it and it + 1 (the two LDS buffers).  The loops run an even
  // number of iterations: an iteration past the last one only stages (its
  // keys are after every query, so no wave computes), which keeps the
  // bodies free of exits between the two halves.
  auto pair = [&](auto masked, int it) __attribute__((always_inline)) {
    stage(0, kr0, vr0);
    const uint32_t okA = ok0;
    __syncthreads();
    ok0 = fetch(ids, kr0, vr0);
    load_ids(it + 3, ids);
    step(masked, it, 0, okA);
    stage(1, kr1, vr1);
    const uint32_t okB = ok1;
    __syncthreads();
    ok1 = fetch(ids, kr1, vr1);
    load_ids(it + 4, ids);
    step(masked, it + 1, 1, okB);
  };
  // First the pairs whose keys are all valid and at or before the wave's
  // first query (no mask), then the rest with the mask.  The switch point is
  // per wave (wave-uniform); both loops pass the same barriers, so the waves
  // of the workgroup stay in step.  Separate loops, not a branch per
  // iteration, keep the two variants' registers apart.
  constexpr uint32_t kAllValid = (1u << KB) - 1u;
  const int nit2 = (nit + 1) & ~1;
  int it = 0;
  for (; it < nit2; it += 2) {
    const int klast = (it + 2 < nit ? it + 2 : nit) * KB * kBS - 1;  // last key of the pair
    const bool plain = !active || (ok0 == kAllValid && (it + 1 >= nit || ok1 == kAllValid) &&
                                   klast <= pos0 + qr0);
    if (!plain) break;
    pair(std::false_type{}, it);
  }
  for (; it < nit2; it += 2) pair(std::true_type{}, it);

  // every lane kept its own keys' sum of the row (rescaled with the row's
  // maximum like the accumulators): the row sum over its four lanes, with
  // every lane of the wave still active for the swaps
#pragma unroll
  for (int hh = 0; hh < HW; ++hh) l[hh] = xor48_sum(l[hh]);
  if constexpr (!STAGE_OUT) {
    if (!row_ok) return;
#pragma unroll
    for (int hh = 0; hh < HW; ++hh) {
      const float inv = l[hh] > 0.0f ? 1.0f / l[hh] : 0.0f;
      float* op = out + ((int64_t)(s0 + qi) * num_q_heads + h0 + hh) * D + 4 * grp;
#pragma unroll
      for (int c = 0; c < NO; ++c)
        // nontemporal: the rows are not read again by this kernel
        __builtin_nontemporal_store(
            f32x4_t{o[hh][c][0] * inv, o[hh][c][1] * inv, o[hh][c][2] * inv, o[hh][c][3] * inv},
            reinterpret_cast<f32x4_t*>(op + 16 * c));
    }
  } else {
    // The output through the wave's own LDS rows (outside the staging
    // buffers), head by head: lane (grp, r16) holds dims 16 c + 4 grp .. + 3
    // of row r16; the rows go out whole, unit u on lane u % 64.
    auto wave_sync = []() __attribute__((always_inline)) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    constexpr int UPO = D / 4;               // 16-byte units per output row
    constexpr int OU = 16 * UPO / 64;        // units per lane and head
    static_assert((16 * UPO) % 64 == 0, "whole units per lane");
    float* orows = reinterpret_cast<float*>(s_raw + KV_BYTES) + w * 16 * RWO;
#pragma unroll
    for (int hh = 0; hh < HW; ++hh) {
      const float inv = l[hh] > 0.0f ? 1.0f / l[hh] : 0.0f;
#pragma unroll
      for (int c = 0; c < NO; ++c)
        *reinterpret_cast<float4*>(orows + r16 * RWO + 16 * c + 4 * grp) =
            make_float4(o[hh][c][0] * inv, o[hh][c][1] * inv, o[hh][c][2] * inv, o[hh][c][3] * inv);
      wave_sync();
      // all of the head's rows read back first, then stored: a store's data
      // registers are then never reused while stores are in flight (which
      // would wait for the stores to complete)
      f32x4_t orow[OU];
#pragma unroll
      for (int k = 0; k < OU; ++k) {
        const int u = lane + 64 * k;
        orow[k] = *reinterpret_cast<const f32x4_t*>(orows + (u / UPO) * RWO + (u % UPO) * 4);
      }
      wave_sync();  // read before the next head overwrites
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < OU; ++k) {
        const int u = lane + 64 * k, row = u / UPO, col = (u % UPO) * 4;
        // nontemporal: the rows are not read again by this kernel (the
        // admissions, whose fp32 output is ~45% of their bytes, ran 4% faster)
        if (qr0 + row < nr)
          __builtin_nontemporal_store(
              orow[k], reinterpret_cast<f32x4_t*>(
                           out + ((int64_t)(s0 + qr0 + row) * num_q_heads + h0 + hh) * D + col));
      }
    }
  }
  if constexpr (PFN) {
#pragma unroll
    for (int i = 0; i < PF; ++i) asm volatile("" ::"v"(pfv[i]));
  }
}

using PrefillFn = void (*)(float*, const float*, const void*, const void*, const int32_t*, int,
                           const int32_t*, const int32_t*, int, int64_t, int, float, int, int, int);

// Waves per workgroup, query heads per wave (for groups of at least 4 heads)
// and key blocks per staged iteration.  With 8 waves a workgroup may hold up
// to 256 VGPRs per lane, which two heads per wave need at D = 128.
#ifndef RKV_PREFILL_WAVES
#define RKV_PREFILL_WAVES 8
#endif
#ifndef RKV_PREFILL_HW
#define RKV_PREFILL_HW 2
#endif
#ifndef RKV_PREFILL_KB
#define RKV_PREFILL_KB 2
#endif
// Heaviest query tiles first (1) or the query tile as the fastest grid
// dimension (0).
#ifndef RKV_PREFILL_HEAVY_FIRST
#define RKV_PREFILL_HEAVY_FIRST 1
#endif
// A build of RKV_PREFILL_SHORT_WAVES waves per workgroup that touches the
// q rows of the next round's workgroups (RKV_PREFILL_PREFETCH), for bf16
// pools on the calls short_build_use (below) gives it: G = 4 -> 32-row
// tiles, G = 8 -> 16-row, G = 2 -> 32-row, G = 1 -> 64-row; at D = 128 and
// G >= 4 two workgroups per CU (235 VGPRs, 68 KB of LDS), at D = 64 three.
// Where it loses, the 8-wave tiles, which stage each K/V tile for twice the
// rows, stay.  us per call (one box, interleaved; 8-wave -> 4-wave) for 25 x
// 128 new tokens / 8 x 512 square / 8 x 512 after 512 cached / after 3584
// cached: G = 4, D = 128: 29.8 -> 26.0 / 52.6 -> 51.5 / 104 = 104 / 413 ->
// 430; G = 8, D = 128: 64.3 -> 61.4 / 109 -> 100 / 215 = 215 / 827 -> 849;
// G = 2, D = 128: 17.4 -> 19.7 / 31.5 -> 33.3 / 57.8 -> 66.0 / 224 -> 261;
// G = 1, D = 128: 13.2 -> 11.6 / 25.8 -> 21.9 / 42.6 -> 38.6 / 144 = 143;
// D = 64, G = 8, 4, 2, 1: 35.1 -> 26.4, 19.5 -> 16.6, 10.9 = 10.8, 8.1 ->
// 7.2 / 67.9 -> 52.7, 34.8 -> 30.2, 22.2 -> 19.3, 18.4 -> 14.4 / -, 69.9 ->
// 62.5, 38.7 -> 35.3, 30.9 -> 25.4 / 535 -> 486, 270 -> 265, 144 = 145,
// 103 -> 93; D = 32, G = 8, 4, 2, 1: 16.5 = 16.3, 10.9 = 11.0, 7.5 = 7.6,
// 6.0 -> 5.8 / 34.9 = 34.6, 22.0 -> 20.4, 15.4 -> 14.9, 13.4 -> 12.6 /
// 75.7 = 75.5, -, 28.4 -> 27.1, 23.3 -> 22.1 / 307 -> 314, 166 -> 173, 104
// -> 107, 85.5 -> 83.3.
#ifndef RKV_PREFILL_SHORT_WAVES
#define RKV_PREFILL_SHORT_WAVES 4
#endif
#ifndef RKV_PREFILL_PREFETCH
#define RKV_PREFILL_PREFETCH 1
#endif
constexpr int kWaves = RKV_PREFILL_WAVES;
constexpr int kShortWaves = RKV_PREFILL_SHORT_WAVES;
constexpr int kHW = RKV_PREFILL_HW;
constexpr int kKB = RKV_PREFILL_KB;

struct PrefillCfg {
  PrefillFn fn;
  int waves;   // per workgroup
  int tile;    // query tokens per workgroup
  bool next;   // touches the next round's q rows (wants pf_stride)
};

// Workgroups of fn (threads each) resident on the current device at once:
// compute units x workgroups per compute unit, asked of the runtime once per
// (device, kernel) and kept; 0 if the runtime cannot say.
int resident_workgroups(PrefillFn fn, int threads) {
  struct Entry {
    PrefillFn fn;
    int device, resident;
  };
  static std::mutex mu;
  static Entry table[256];
  static int used = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i)
    if (table[i].fn == fn && table[i].device == dev) return table[i].resident;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(fn),
                                                   threads, 0) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  const int resident = cus * per_cu;
  if (used < 256) table[used++] = {fn, dev, resident};
  return resident;
}

template <typename T, int D, int G, int W, bool PFN>
PrefillCfg cfg_g() {
  constexpr int HW = G >= 4 && G % kHW == 0 ? kHW : 1;
  constexpr int QS = W / (G / HW) > 0 ? W / (G / HW) : 1;  // row sub-tiles
  return {&prefill_kernel<T, D, G, HW, QS, kKB, PFN>, (G / HW) * QS, 16 * QS, PFN};
}

// When the 4-wave build is taken: 2 on every call, 1 when the sequences
// hold at most as many cached keys as new tokens, 0 never.  fp32 pools (us
// per call, same four shapes as above; 8-wave -> 4-wave): G = 1, D = 32
// 6.2 -> 5.8 / 14.5 -> 13.2 / 25.2 -> 23.2 / 95 -> 83; G = 1, D = 128 15.4
// -> 14.8 / 32.4 -> 30.7 / 57.2 = 58.4 / 219 -> 242; elsewhere slower or
// even (G = 4, D = 32: 11.6 = 11.6 / 25.0 -> 23.3 / 50.9 -> 52.2 / 209 ->
// 226; at D = 64 slower on all four; at D = 128 and G >= 4 the 4-wave form
// spills into AGPRs at one wave per SIMD).
constexpr int short_build_use(bool f32, int G, int D) {
  if (f32) return G == 1 && D == 32 ? 2 : G == 1 && D == 128 ? 1 : 0;
  return D == 64 ? 2 : G == 1 ? 2 : (D == 128 && G == 2) ? 0 : 1;
}

template <typename T, int D, int G>
PrefillCfg cfg_pick(bool short_prefix) {
  constexpr int use = short_build_use(sizeof(T) == 4, G, D);
  if constexpr (use > 0)
    if (use == 2 || short_prefix) return cfg_g<T, D, G, kShortWaves, RKV_PREFILL_PREFETCH != 0>();
  return cfg_g<T, D, G, kWaves, false>();
}

template <typename T, int D>
PrefillCfg pick_g(int G, bool short_prefix) {
  switch (G) {
    case 1: return cfg_pick<T, D, 1>(short_prefix);
    case 2: return cfg_pick<T, D, 2>(short_prefix);
    case 4: return cfg_pick<T, D, 4>(short_prefix);
    case 8: return cfg_pick<T, D, 8>(short_prefix);
    default: return {nullptr, 0, 0, false};
  }
}

template <typename T>
PrefillCfg pick_d(int D, int G, bool short_prefix) {
  switch (D) {
    case 32: return pick_g<T, 32>(G, short_prefix);
    case 64: return pick_g<T, 64>(G, short_prefix);
    case 128: return pick_g<T, 128>(G, short_prefix);
    default: return {nullptr, 0, 0, false};
  }
}

}  // namespace
}  // namespace rkv

using namespace rkv;

extern "C" int rkv_prefill_attention(float* out, const float* q, const void* k_pool,
                                     const void* v_pool, const int32_t* block_tables,
                                     int max_blocks_per_seq, const int32_t* q_start,
                                     const int32_t* ctx_lens, int num_seqs, int num_q_heads,
                                     int num_kv_heads, int head_dim, int block_size,
                                     int64_t num_blocks, int max_q_len, float scale, int dtype,
                                     void* stream) {
  clear_error();
  if (num_seqs < 0 || max_blocks_per_seq < 0 || num_blocks < 0 || max_q_len < 0)
    return fail(RKV_ERR_INVALID_ARG, "rkv_prefill_attention: negative size argument");
  if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads)
    return fail(RKV_ERR_INVALID_ARG,
                "rkv_prefill_attention: num_q_heads must be a positive multiple of num_kv_heads");
  if (dtype != RKV_F32 && dtype != RKV_BF16)
    return fail(RKV_ERR_INVALID_ARG, "rkv_prefill_attention: dtype must be RKV_F32 or RKV_BF16");
  if (block_size != kBS)
    return fail(RKV_ERR_UNSUPPORTED, "rkv_prefill_attention: block_size must be 16");
  const int G = num_q_heads / num_kv_heads;
  // at most as many cached keys as new tokens, judged by the table width
  // (the keys a sequence can hold) against the longest new-token run
  const bool short_prefix = (int64_t)max_blocks_per_seq * kBS <= 2 * (int64_t)max_q_len;
  const PrefillCfg cfg = dtype == RKV_BF16 ? pick_d<uint16_t>(head_dim, G, short_prefix)
                                           : pick_d<float>(head_dim, G, short_prefix);
  if (!cfg.fn)
    return fail(RKV_ERR_UNSUPPORTED,
                "rkv_prefill_attention: head_dim must be 32, 64 or 128 and num_q_heads / "
                "num_kv_heads 1, 2, 4 or 8");
  if (num_seqs > 65535 || num_kv_heads > 65535)
    return fail(RKV_ERR_INVALID_ARG,
                "rkv_prefill_attention: num_seqs and num_kv_heads must be <= 65535");
  if (num_seqs == 0 || max_q_len == 0 || max_blocks_per_seq == 0) return RKV_OK;
  if ((int64_t)max_blocks_per_seq * kBS > 0x7fffffff)
    return fail(RKV_ERR_INVALID_ARG, "rkv_prefill_attention: max_blocks_per_seq too large");
  if (num_blocks < 1) return fail(RKV_ERR_INVALID_ARG, "rkv_prefill_attention: num_blocks < 1");
  if (!out || !q || !k_pool || !v_pool || !block_tables || !q_start || !ctx_lens)
    return fail(RKV_ERR_INVALID_ARG, "rkv_prefill_attention: null pointer argument");
  if (!aligned16(out) || !aligned16(q) || !aligned16(k_pool) || !aligned16(v_pool))
    return fail(RKV_ERR_INVALID_ARG,
                "rkv_prefill_attention: out, q and pools must be 16-byte aligned");
  const int64_t n_tiles = (max_q_len + cfg.tile - 1) / cfg.tile;
  const int64_t n_heads = (int64_t)num_seqs * num_kv_heads;
  const int heavy = RKV_PREFILL_HEAVY_FIRST && n_tiles <= 65535 && n_heads <= 0x7fffffff;
  const dim3 grid = heavy ? dim3((unsigned)n_heads, (unsigned)n_tiles, 1)
                          : dim3((unsigned)n_tiles, (unsigned)num_kv_heads, (unsigned)num_seqs);
  // Of R resident workgroups and T in all, the later ones (from R on) start
  // as slots free up.  The touches go to the last min(R, T - R) workgroups
  // of the first round (its lightest: the grid runs heaviest first), each
  // for the workgroup that many places later; the heaviest, which end the
  // first round, touch nothing.  configs[4] admissions (us per call, one
  // box, interleaved): 26.7 against 28.6 when the first T - R workgroups
  // touch and 27.4 when the first R - (T - R) touch workgroups of the first
  // round (8 x 512 square: the same workgroups either way, 52.6).
  int pf_stride = 0, pf_first = 0;
  if (cfg.next && heavy) {
    const int64_t R = resident_workgroups(cfg.fn, 64 * cfg.waves), T = n_heads * n_tiles;
    if (R > 0 && T > R) {
      pf_stride = (int)(T - R < R ? T - R : R);
      pf_first = (int)(R - pf_stride);
    }
  }
  hipLaunchKernelGGL(cfg.fn, grid, dim3(64 * cfg.waves), 0, static_cast<hipStream_t>(stream), out, q, k_pool,
                     v_pool, block_tables, max_blocks_per_seq, q_start, ctx_lens, num_kv_heads,
                     num_blocks, max_q_len, scale * kLog2e, heavy, pf_stride, pf_first);
  return check_launch("rkv_prefill_attention");
}
