// device_blocks.hip -- the paged block manager with its state in HBM: the
// FIFO free list (a ring of block ids), the block tables and their lengths.
// A decode step can then grow the tables, map token positions to pool slots,
// append and attend without a host round trip (and be captured in a HIP
// graph).  The semantics are those of the host manager (rkv_bm_*, after
// PagedCache, crates/nn/src/kv_cache.rs:381-432): ids leave from the front of
// the free list and are appended to a sequence's table; freed ids return to
// the back in table order.  One call over n sequences equals n host calls in
// the same order (ids are handed out by a prefix sum in call order), except
// that a reserve is all-or-nothing: when the pool cannot cover every
// sequence of the call, nothing is taken and the error flag says OOM.
//
// Each operation is one workgroup (1024 threads) walking the call's
// sequences in chunks with a block-wide prefix sum; the ring position of the
// front / back and the error flag live in a small control record that only
// these kernels touch, in stream order.
#include "common.hpp"

#include "../../include/rustral_serving.h"

namespace rkv {
namespace {

constexpr int kThreads = 1024;

struct Ctl {
  int64_t head;  // ring position of the front of the free list
  int64_t tail;  // ring position one past its back (free = tail - head)
  int32_t err;   // RKV_DBM_ERR_* of the last failed call (sticky until read)
  int32_t pad;
};

// Set in a sequence's length while a call checks its slots for repeats
// (lengths stay below it: max_blocks_per_seq < 2^30).
constexpr int32_t kMark = 1 << 30;

// Flags RKV_DBM_ERR_ARG in *bad when a slot occurs twice in slots[0, n): each
// thread sets the mark bit of its slot's length, and a mark already set means
// an earlier occurrence; then clears the marks again.  Slots outside
// [0, max_seqs) are left to the caller's own check.
__device__ void find_repeats(int32_t* __restrict__ nblk, const int32_t* __restrict__ slots,
                             int n, int max_seqs, int* bad) {
  const int t = threadIdx.x;
  for (int i = t; i < n; i += kThreads) {
    const int s = slots[i];
    if (s >= 0 && s < max_seqs && (atomicOr(&nblk[s], kMark) & kMark))
      atomicOr(bad, RKV_DBM_ERR_ARG);
  }
  __syncthreads();
  for (int i = t; i < n; i += kThreads) {
    const int s = slots[i];
    if (s >= 0 && s < max_seqs) atomicAnd(&nblk[s], ~kMark);
  }
  __syncthreads();
}

// Exclusive prefix sum of v over the workgroup (kThreads values); returns the
// thread's offset and the chunk total in *total.
__device__ int64_t block_scan(int64_t v, int64_t* s, int64_t* total) {
  const int t = threadIdx.x;
  s[t] = v;
  __syncthreads();
  for (int o = 1; o < kThreads; o <<= 1) {
    const int64_t x = t >= o ? s[t - o] : 0;
    __syncthreads();
    s[t] += x;
    __syncthreads();
  }
  const int64_t incl = s[t];
  *total = s[kThreads - 1];
  __syncthreads();
  return incl - v;
}

__global__ void init_kernel(int32_t* ring, int32_t* tables, int32_t* nblk, Ctl* ctl,
                            int64_t num_blocks, int64_t table_elems, int max_seqs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t x = i; x < num_blocks; x += stride) ring[x] = (int32_t)x;
  for (int64_t x = i; x < table_elems; x += stride) tables[x] = -1;
  for (int64_t x = i; x < max_seqs; x += stride) nblk[x] = 0;
  if (i == 0) {
    ctl->head = 0;
    ctl->tail = num_blocks;
    ctl->err = 0;
    ctl->pad = 0;
  }
}

// Grows the table of slots[i] to ceil(num_tokens[i] / bs) blocks, i in call
// order; all-or-nothing.
__global__ __launch_bounds__(kThreads) void reserve_kernel(
    int32_t* __restrict__ ring, int32_t* __restrict__ tables, int32_t* __restrict__ nblk,
    Ctl* __restrict__ ctl, const int32_t* __restrict__ slots,
    const int32_t* __restrict__ num_tokens, int n, int64_t num_blocks, int max_seqs,
    int max_blocks, int bs) {
  __shared__ int64_t s_scan[kThreads];
  __shared__ int s_bad;
  const int t = threadIdx.x;
  if (t == 0) s_bad = 0;
  __syncthreads();
  find_repeats(nblk, slots, n, max_seqs, &s_bad);
  // pass 1: validate and count
  int64_t need_all = 0;
  for (int c0 = 0; c0 < n; c0 += kThreads) {
    const int i = c0 + t;
    int64_t need = 0;
    if (i < n) {
      const int s = slots[i], nt = num_tokens[i];
      if (s < 0 || s >= max_seqs || nt < 0) {
        atomicOr(&s_bad, RKV_DBM_ERR_ARG);
      } else {
        const int64_t want = ((int64_t)nt + bs - 1) / bs;
        if (want > max_blocks) atomicOr(&s_bad, RKV_DBM_ERR_TABLE_FULL);
        else need = want > nblk[s] ? want - nblk[s] : 0;
      }
    }
    int64_t tot;
    block_scan(need, s_scan, &tot);
    need_all += tot;
  }
  const int64_t head = ctl->head, avail = ctl->tail - head;
  const int bad = s_bad | (need_all > avail ? RKV_DBM_ERR_OOM : 0);
  if (bad) {
    if (t == 0) ctl->err = bad;
    return;
  }
  // pass 2: hand out ids in call order
  int64_t base = 0;
  for (int c0 = 0; c0 < n; c0 += kThreads) {
    const int i = c0 + t;
    int s = 0, have = 0;
    int64_t need = 0;
    if (i < n) {
      s = slots[i];
      have = nblk[s];
      const int64_t want = ((int64_t)num_tokens[i] + bs - 1) / bs;
      need = want > have ? want - have : 0;
    }
    int64_t tot;
    const int64_t off = block_scan(need, s_scan, &tot);
    for (int64_t k = 0; k < need; ++k)
      tables[(int64_t)s * max_blocks + have + k] = ring[(head + base + off + k) % num_blocks];
    if (need > 0) nblk[s] = have + (int)need;
    base += tot;
  }
  __syncthreads();
  if (t == 0) ctl->head = head + base;
}

// Returns every block of slots[i] to the back of the free list (table
// order, i in call order) and empties the tables.
__global__ __launch_bounds__(kThreads) void free_kernel(
    int32_t* __restrict__ ring, int32_t* __restrict__ tables, int32_t* __restrict__ nblk,
    Ctl* __restrict__ ctl, const int32_t* __restrict__ slots, int n, int64_t num_blocks,
    int max_seqs, int max_blocks) {
  __shared__ int64_t s_scan[kThreads];
  __shared__ int s_bad;
  const int t = threadIdx.x;
  if (t == 0) s_bad = 0;
  __syncthreads();
  find_repeats(nblk, slots, n, max_seqs, &s_bad);
  for (int c0 = 0; c0 < n; c0 += kThreads) {
    const int i = c0 + t;
    if (i < n && (slots[i] < 0 || slots[i] >= max_seqs)) atomicOr(&s_bad, RKV_DBM_ERR_ARG);
  }
  __syncthreads();
  if (s_bad) {
    if (t == 0) ctl->err = s_bad;
    return;
  }
  const int64_t tail = ctl->tail;
  int64_t base = 0;
  for (int c0 = 0; c0 < n; c0 += kThreads) {
    const int i = c0 + t;
    const int s = i < n ? slots[i] : 0;
    const int64_t cnt = i < n ? nblk[s] : 0;
    int64_t tot;
    const int64_t off = block_scan(cnt, s_scan, &tot);
    int32_t* row = tables + (int64_t)s * max_blocks;
    for (int64_t k = 0; k < cnt; ++k) {
      ring[(tail + base + off + k) % num_blocks] = row[k];
      row[k] = -1;
    }
    if (i < n) nblk[s] = 0;
    base += tot;
  }
  __syncthreads();
  if (t == 0) ctl->tail = tail + base;
}

// slots_out[i] = the pool slot of token position positions[i] of slots[i]
// (block id * bs + offset), or -1 when the table does not cover it.
__global__ void slot_mapping_kernel(const int32_t* __restrict__ tables,
                                    const int32_t* __restrict__ nblk,
                                    const int32_t* __restrict__ slots,
                                    const int32_t* __restrict__ positions,
                                    int64_t* __restrict__ out, int n, int max_seqs,
                                    int max_blocks, int bs) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int s = slots[i], p = positions[i];
  int64_t r = -1;
  if (s >= 0 && s < max_seqs && p >= 0 && p / bs < nblk[s])
    r = (int64_t)tables[(int64_t)s * max_blocks + p / bs] * bs + p % bs;
  out[i] = r;
}

// out[i][j] = table of slots[i] (j < out_width; -1 past its length).
__global__ void batch_tables_kernel(const int32_t* __restrict__ tables,
                                    const int32_t* __restrict__ nblk,
                                    const int32_t* __restrict__ slots,
                                    int32_t* __restrict__ out, int n, int out_width,
                                    int max_seqs, int max_blocks) {
  const int i = blockIdx.y;
  const int s = slots[i];
  const bool ok = s >= 0 && s < max_seqs;
  const int len = ok ? nblk[s] : 0;
  for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < out_width;
       j += gridDim.x * blockDim.x)
    out[(int64_t)i * out_width + j] = j < len ? tables[(int64_t)s * max_blocks + j] : -1;
}

}  // namespace
}  // namespace rkv

using namespace rkv;

struct rkv_device_block_manager {
  int64_t num_blocks = 0;
  int block_size = 0, max_seqs = 0, max_blocks = 0;
  int32_t* ring = nullptr;
  int32_t* tables = nullptr;
  int32_t* nblk = nullptr;
  Ctl* ctl = nullptr;
};

static void dbm_release(rkv_device_block_manager* bm) {
  if (!bm) return;
  if (bm->ring) (void)hipFree(bm->ring);
  if (bm->tables) (void)hipFree(bm->tables);
  if (bm->nblk) (void)hipFree(bm->nblk);
  if (bm->ctl) (void)hipFree(bm->ctl);
  delete bm;
}

extern "C" rkv_device_block_manager* rkv_dbm_create(int64_t num_blocks, int block_size,
                                                    int max_seqs, int max_blocks_per_seq,
                                                    void* stream) {
  clear_error();
  if (num_blocks < 1 || num_blocks > 0x7fffffff || block_size < 1 || max_seqs < 1 ||
      max_blocks_per_seq < 1 || max_blocks_per_seq >= kMark) {
    fail(RKV_ERR_INVALID_ARG, "rkv_dbm_create: bad argument");
    return nullptr;
  }
  auto* bm = new rkv_device_block_manager;
  bm->num_blocks = num_blocks;
  bm->block_size = block_size;
  bm->max_seqs = max_seqs;
  bm->max_blocks = max_blocks_per_seq;
  const int64_t table_elems = (int64_t)max_seqs * max_blocks_per_seq;
  if (hipMalloc(&bm->ring, num_blocks * sizeof(int32_t)) != hipSuccess ||
      hipMalloc(&bm->tables, table_elems * sizeof(int32_t)) != hipSuccess ||
      hipMalloc(&bm->nblk, max_seqs * sizeof(int32_t)) != hipSuccess ||
      hipMalloc(&bm->ctl, sizeof(Ctl)) != hipSuccess) {
    (void)hipGetLastError();
    dbm_release(bm);
    fail(RKV_ERR_HIP, "rkv_dbm_create: device allocation failed");
    return nullptr;
  }
  const int64_t most = num_blocks > table_elems ? num_blocks : table_elems;
  const int grid = (int)((most + 255) / 256 < 4096 ? (most + 255) / 256 : 4096);
  hipLaunchKernelGGL(init_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     bm->ring, bm->tables, bm->nblk, bm->ctl, num_blocks, table_elems, max_seqs);
  if (check_launch("rkv_dbm_create")) {
    dbm_release(bm);
    return nullptr;
  }
  return bm;
}

extern "C" void rkv_dbm_destroy(rkv_device_block_manager* bm) { dbm_release(bm); }

extern "C" int rkv_dbm_reserve(rkv_device_block_manager* bm, const int32_t* slots,
                               const int32_t* num_tokens, int n, void* stream) {
  clear_error();
  if (!bm || n < 0) return fail(RKV_ERR_INVALID_ARG, "rkv_dbm_reserve: bad argument");
  if (n == 0) return RKV_OK;
  if (!slots || !num_tokens) return fail(RKV_ERR_INVALID_ARG, "rkv_dbm_reserve: null pointer");
  hipLaunchKernelGGL(reserve_kernel, dim3(1), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     bm->ring, bm->tables, bm->nblk, bm->ctl, slots, num_tokens, n,
                     bm->num_blocks, bm->max_seqs, bm->max_blocks, bm->block_size);
  return check_launch("rkv_dbm_reserve");
}

extern "C" int rkv_dbm_free(rkv_device_block_manager* bm, const int32_t* slots, int n,
                            void* stream) {
  clear_error();
  if (!bm || n < 0) return fail(RKV_ERR_INVALID_ARG, "rkv_dbm_free: bad argument");
  if (n == 0) return RKV_OK;
  if (!slots) return fail(RKV_ERR_INVALID_ARG, "rkv_dbm_free: null pointer");
  hipLaunchKernelGGL(free_kernel, dim3(1), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     bm->ring, bm->tables, bm->nblk, bm->ctl, slots, n, bm->num_blocks,
                     bm->max_seqs, bm->max_blocks);
  return check_launch("rkv_dbm_free");
}

extern "C" int rkv_dbm_slot_mapping(const rkv_device_block_manager* bm, const int32_t* slots,
                                    const int32_t* positions, int n, int64_t* slot_mapping,
                                    void* stream) {
  clear_error();
  if (!bm || n < 0) return fail(RKV_ERR_INVALID_ARG, "rkv_dbm_slot_mapping: bad argument");
  if (n == 0) return RKV_OK;
  if (!slots || !positions || !slot_mapping)
    return fail(RKV_ERR_INVALID_ARG, "rkv_dbm_slot_mapping: null pointer");
  hipLaunchKernelGGL(slot_mapping_kernel, dim3((n + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), bm->tables, bm->nblk, slots, positions,
                     slot_mapping, n, bm->max_seqs, bm->max_blocks, bm->block_size);
  return check_launch("rkv_dbm_slot_mapping");
}

extern "C" int rkv_dbm_batch_tables(const rkv_device_block_manager* bm, const int32_t* slots,
                                    int n, int32_t* tables, int max_blocks, void* stream) {
  clear_error();
  if (!bm || n < 0 || max_blocks < 1 || n > 65535)
    return fail(RKV_ERR_INVALID_ARG, "rkv_dbm_batch_tables: bad argument");
  if (n == 0) return RKV_OK;
  if (!slots || !tables) return fail(RKV_ERR_INVALID_ARG, "rkv_dbm_batch_tables: null pointer");
  const int gx = (max_blocks + 255) / 256 < 64 ? (max_blocks + 255) / 256 : 64;
  hipLaunchKernelGGL(batch_tables_kernel, dim3(gx, n), dim3(256), 0,
                     static_cast<hipStream_t>(stream), bm->tables, bm->nblk, slots, tables, n,
                     max_blocks, bm->max_seqs, bm->max_blocks);
  return check_launch("rkv_dbm_batch_tables");
}

extern "C" int rkv_dbm_status(rkv_device_block_manager* bm, int64_t* num_free, int32_t* err,
                              int clear, void* stream) {
  clear_error();
  if (!bm) return fail(RKV_ERR_INVALID_ARG, "rkv_dbm_status: bad argument");
  Ctl c{};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (hipMemcpyAsync(&c, bm->ctl, sizeof(Ctl), hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return fail(RKV_ERR_HIP, "rkv_dbm_status: copy failed");
  if (num_free) *num_free = c.tail - c.head;
  if (err) *err = c.err;
  if (clear && c.err) {
    // cleared by a small copy of the zeroed field (no memset node)
    const int32_t zero = 0;
    if (hipMemcpyAsync(reinterpret_cast<char*>(bm->ctl) + offsetof(Ctl, err), &zero,
                       sizeof(zero), hipMemcpyHostToDevice, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
      return fail(RKV_ERR_HIP, "rkv_dbm_status: clear failed");
  }
  return RKV_OK;
}

extern "C" int rkv_dbm_download(const rkv_device_block_manager* bm, int32_t* tables,
                                int32_t* lengths, int32_t* free_list, int64_t* num_free,
                                void* stream) {
  clear_error();
  if (!bm) return fail(RKV_ERR_INVALID_ARG, "rkv_dbm_download: bad argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  Ctl c{};
  if (hipMemcpyAsync(&c, bm->ctl, sizeof(Ctl), hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return fail(RKV_ERR_HIP, "rkv_dbm_download: copy failed");
  const int64_t te = (int64_t)bm->max_seqs * bm->max_blocks;
  if (tables && hipMemcpyAsync(tables, bm->tables, te * sizeof(int32_t), hipMemcpyDeviceToHost,
                               st) != hipSuccess)
    return fail(RKV_ERR_HIP, "rkv_dbm_download: copy failed");
  if (lengths && hipMemcpyAsync(lengths, bm->nblk, bm->max_seqs * sizeof(int32_t),
                                hipMemcpyDeviceToHost, st) != hipSuccess)
    return fail(RKV_ERR_HIP, "rkv_dbm_download: copy failed");
  const int64_t nf = c.tail - c.head;
  if (free_list && nf > 0) {
    // front first: ring positions head .. tail - 1 (at most two pieces)
    const int64_t h = c.head % bm->num_blocks;
    const int64_t first = nf < bm->num_blocks - h ? nf : bm->num_blocks - h;
    if (hipMemcpyAsync(free_list, bm->ring + h, first * sizeof(int32_t), hipMemcpyDeviceToHost,
                       st) != hipSuccess ||
        (nf > first && hipMemcpyAsync(free_list + first, bm->ring, (nf - first) * sizeof(int32_t),
                                      hipMemcpyDeviceToHost, st) != hipSuccess))
      return fail(RKV_ERR_HIP, "rkv_dbm_download: copy failed");
  }
  if (hipStreamSynchronize(st) != hipSuccess)
    return fail(RKV_ERR_HIP, "rkv_dbm_download: synchronize failed");
  if (num_free) *num_free = nf;
  return RKV_OK;
}
