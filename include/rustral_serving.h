/*
 * rustral_serving.h -- paged block manager (host-side and device-side) and
 * continuous-batching scheduler of librustral_kv.so (plain C ABI; the
 * rkv_bm_* / rkv_sched_* handles keep their state in host memory, the
 * rkv_dbm_* manager in device memory).
 *
 * These are the callers of the device path: the block manager hands out the
 * block ids that rkv_append / rkv_gather / rkv_decode_attention index, and
 * plans the compaction moves rkv_copy_blocks executes; the scheduler builds
 * each step's batch (sequence lengths + block tables) from requests.
 *
 * Return codes and rkv_last_error() are those of rustral_kv.h.  Handles are
 * not thread-safe: one handle is used by one thread at a time (the
 * reference types are plain owned structs, &mut self).
 */
#ifndef RUSTRAL_SERVING_H
#define RUSTRAL_SERVING_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RKV_ERR_OOM (-5) /* KV pool exhausted: PagedCache::allocate's None,
                            Scheduler::update's CoreError::Other("KV cache out of memory") */

/* ---- block manager (PagedCache) ------------------------------------------ */

typedef struct rkv_block_manager rkv_block_manager;

/* Replaces PagedCache::new (crates/nn/src/kv_cache.rs:399-411): block ids
 * 0..num_blocks-1 start on a FIFO free list in ascending order.  NULL on bad
 * arguments (see rkv_last_error). */
rkv_block_manager* rkv_bm_create(int64_t num_blocks, int block_size);
void rkv_bm_destroy(rkv_block_manager* bm);

/* Replaces PagedCache::allocate (kv_cache.rs:413-425): takes
 * ceil(num_tokens / block_size) ids from the FRONT of the free list and
 * APPENDS them to seq_id's block table (the reference overwrites the table,
 * which leaks the earlier blocks; kv_cache.rs:422).  Returns the number of
 * blocks taken (>= 0) and copies their ids to out_ids when out_ids != NULL
 * (at most cap of them), or RKV_ERR_OOM (nothing taken) when fewer blocks
 * are free, mirroring the reference's None. */
int64_t rkv_bm_allocate(rkv_block_manager* bm, int64_t seq_id, int64_t num_tokens,
                        int32_t* out_ids, int64_t cap);

/* Grows seq_id's table to ceil(num_tokens / block_size) blocks (allocating
 * only the missing ones).  Returns the number of blocks added or RKV_ERR_OOM. */
int64_t rkv_bm_reserve(rkv_block_manager* bm, int64_t seq_id, int64_t num_tokens);

/* Replaces PagedCache::free (kv_cache.rs:427-431): the sequence's blocks go
 * to the BACK of the free list, in table order.  Returns how many (0 for an
 * unknown sequence). */
int64_t rkv_bm_free(rkv_block_manager* bm, int64_t seq_id);

int64_t rkv_bm_num_free(const rkv_block_manager* bm);
int64_t rkv_bm_num_blocks(const rkv_block_manager* bm);
int rkv_bm_block_size(const rkv_block_manager* bm);

/* Copies seq_id's block table (at most cap ids) to out; returns its length
 * (0 for an unknown sequence). */
int64_t rkv_bm_table(const rkv_block_manager* bm, int64_t seq_id, int32_t* out, int64_t cap);

/* Copies the free list, front first (at most cap ids); returns its length. */
int64_t rkv_bm_free_list(const rkv_block_manager* bm, int32_t* out, int64_t cap);

/* Fills a dense int32 table [n_seqs, max_blocks] for rkv_decode_attention /
 * rkv_gather from the given sequences (missing entries = -1).  Fails with
 * RKV_ERR_INVALID_ARG if a table is longer than max_blocks. */
int rkv_bm_fill_tables(const rkv_block_manager* bm, const int64_t* seq_ids, int n_seqs,
                       int32_t* tables, int max_blocks);

/* Compaction plan (no reference counterpart: the reference's eviction only
 * frees ids, crates/nn/src/continuous_batching.rs:380-386).  Moves up to
 * max_moves live blocks, highest id first, into the lowest free ids below
 * them; rewrites the owning tables; writes the (src, dst) pairs to pairs
 * ([2 * n], for rkv_copy_blocks, which must run before any block is reused)
 * and returns n.  Sources and destinations are disjoint.  Afterwards the free
 * list is sorted ascending, so new allocations fill the low end. */
int64_t rkv_bm_plan_compaction(rkv_block_manager* bm, int64_t max_moves, int32_t* pairs,
                               int64_t cap_pairs);

/* Migration plan: the same moves without the stop at the first free id above
 * the source, so exactly min(max_moves, live blocks, free blocks) live
 * blocks move, highest id first, to the lowest free ids -- it drains the top
 * of the pool (a region to release, or the configs[4] step's relocation of a
 * fixed share of the live blocks).  Pairs, tables and free list as for
 * rkv_bm_plan_compaction; sources (live) and destinations (free) are
 * disjoint. */
int64_t rkv_bm_plan_migration(rkv_block_manager* bm, int64_t max_moves, int32_t* pairs,
                              int64_t cap_pairs);

/* Relocation plan: the blocks rkv_bm_plan_migration would move (the
 * min(max_moves, live, free) highest live ids) go into the longest runs of
 * consecutive free ids -- runs longest first, the lower start on ties, each
 * filled from its low end -- and the i-th lowest source to the i-th lowest
 * destination, so the pairs ascend on both sides.  rkv_copy_blocks then
 * writes runs of consecutive blocks, which this part streams faster than
 * scattered destinations (the writes, not the reads, decide a copy's rate).
 * The free list afterwards holds the unused free ids and the vacated
 * sources, sorted ascending.  Pairs and tables as for rkv_bm_plan_migration;
 * sources and destinations are disjoint.  No reference counterpart (the
 * reference only frees, crates/nn/src/continuous_batching.rs:380-386). */
int64_t rkv_bm_plan_relocation(rkv_block_manager* bm, int64_t max_moves, int32_t* pairs,
                               int64_t cap_pairs);

/* ---- device-side block manager ----------------------------------------------
 * The same FIFO manager with its state in device memory: the free list is a
 * ring of block ids, the tables are an int32 [max_seqs][max_blocks_per_seq]
 * array indexed by the caller's sequence slot, the lengths an int32
 * [max_seqs] array.  Calls are enqueued on the stream (no host
 * synchronisation, so a decode step -- reserve, slot mapping, append,
 * attention -- can run from device memory alone and be captured in a HIP
 * graph); arguments named slots / num_tokens / positions / slot_mapping /
 * tables are device pointers.  One call over n sequences hands out ids in
 * call order, as n host calls would (the same ids in the same tables);
 * sequences of one call must be distinct (a repeated slot fails the call
 * with RKV_DBM_ERR_ARG).  Errors found on the device are
 * recorded in a flag read by rkv_dbm_status; the call that fails changes
 * nothing.  No reference counterpart: PagedCache (crates/nn/src/
 * kv_cache.rs:381-432) lives on the host; this is its device-resident form
 * for the serving loop of continuous_batching.rs:516-537. */
typedef struct rkv_device_block_manager rkv_device_block_manager;

#define RKV_DBM_ERR_OOM 1        /* a reserve needed more blocks than are free */
#define RKV_DBM_ERR_TABLE_FULL 2 /* a table would exceed max_blocks_per_seq */
#define RKV_DBM_ERR_ARG 4        /* a slot outside [0, max_seqs), repeated, or a negative count */

/* Allocates the state (device memory) and starts the free list with ids
 * 0..num_blocks-1 in ascending order (initialised on stream).  NULL on bad
 * arguments (max_blocks_per_seq must be below 2^30) or allocation failure
 * (see rkv_last_error). */
rkv_device_block_manager* rkv_dbm_create(int64_t num_blocks, int block_size, int max_seqs,
                                         int max_blocks_per_seq, void* stream);
void rkv_dbm_destroy(rkv_device_block_manager* bm);

/* Grows the table of slots[i] to ceil(num_tokens[i] / block_size) blocks
 * (as rkv_bm_reserve), i in call order.  All or nothing: if the free list
 * cannot cover the whole call, or a table would overflow, nothing changes
 * and the error flag is set. */
int rkv_dbm_reserve(rkv_device_block_manager* bm, const int32_t* slots, const int32_t* num_tokens,
                    int n, void* stream);

/* Returns every block of slots[i] to the back of the free list in table
 * order (as rkv_bm_free), i in call order, and empties the tables. */
int rkv_dbm_free(rkv_device_block_manager* bm, const int32_t* slots, int n, void* stream);

/* slot_mapping[i] = table[slots[i]][positions[i] / block_size] * block_size +
 * positions[i] % block_size, or -1 when the table does not cover the
 * position (rkv_append skips negative slots). */
int rkv_dbm_slot_mapping(const rkv_device_block_manager* bm, const int32_t* slots,
                         const int32_t* positions, int n, int64_t* slot_mapping, void* stream);

/* Dense block tables [n][max_blocks] of the given slots for
 * rkv_decode_attention / rkv_prefill_attention / rkv_gather (-1 past a
 * table's length). */
int rkv_dbm_batch_tables(const rkv_device_block_manager* bm, const int32_t* slots, int n,
                         int32_t* tables, int max_blocks, void* stream);

/* Synchronises the stream and reports the number of free blocks and the
 * error flag (RKV_DBM_ERR_* bits of the last failed call; clear != 0 resets
 * it). */
int rkv_dbm_status(rkv_device_block_manager* bm, int64_t* num_free, int32_t* err, int clear,
                   void* stream);

/* Synchronises and copies the state to host memory (any pointer may be
 * NULL): tables [max_seqs * max_blocks_per_seq], lengths [max_seqs], the
 * free list front first [num_blocks], and its length. */
int rkv_dbm_download(const rkv_device_block_manager* bm, int32_t* tables, int32_t* lengths,
                     int32_t* free_list, int64_t* num_free, void* stream);

/* ---- scheduler (Scheduler / Batch / Request) -------------------------------- */

typedef struct rkv_scheduler rkv_scheduler;

#define RKV_PRIORITY_LOW 0 /* RequestPriority values, continuous_batching.rs:8-14 */
#define RKV_PRIORITY_NORMAL 1
#define RKV_PRIORITY_HIGH 2
#define RKV_PRIORITY_CRITICAL 3

#define RKV_EOS_TOKEN 2 /* Request::should_complete's stop token (continuous_batching.rs:124-129) */

/* Replaces Scheduler::new (continuous_batching.rs:201-219) with its own
 * PagedCache(block_size, num_blocks).  The reference hard-codes a scheduler
 * block size of 16 independent of the cache (:213); here both are
 * block_size.  preemption_threshold is the reference's 0.5. */
rkv_scheduler* rkv_sched_create(int64_t num_blocks, int block_size, int max_batch_size,
                                int max_seq_len);
void rkv_sched_destroy(rkv_scheduler* s);

/* Scheduler::add_request / add_priority_request (:222-246).  Returns the new
 * id (0, 1, 2, ...) or a negative code.  max_seq_len bounds prompt + max_tokens. */
int64_t rkv_sched_add_request(rkv_scheduler* s, const int32_t* prompt, int n_prompt,
                              int max_tokens, int priority);

/* Scheduler::schedule (:248-296): retire finished requests (their blocks are
 * freed -- the reference keeps them), pause a running request whose last
 * update ran out of blocks and still finds none (the "should preempt" of
 * :313-315; it resumes later by recompute, so no batch row ever has a table
 * shorter than its sequence), resume paused ones (re-allocating their
 * blocks; they then recompute prompt + generated), admit pending ones
 * (allocating ceil(prompt / block_size) blocks), preempt a Low-priority
 * request under pressure, and build the batch.  The batch lists running
 * requests in ascending id order (the reference's HashMap order is random).
 * Returns the batch size (0 = the reference's None); the batch is then read
 * with rkv_sched_batch. */
int rkv_sched_schedule(rkv_scheduler* s);

/* Sizes of the current batch: number of requests, total input tokens, and
 * the longest block table. */
int rkv_sched_batch_dims(const rkv_scheduler* s, int* n_requests, int64_t* n_input_tokens,
                         int* max_blocks);

/* Copies the current batch (Batch, :157-167) into caller buffers; any pointer
 * may be NULL.  request_ids [n]; seq_lens [n] (prompt + generated);
 * input_offsets [n + 1] into input_ids [n_input_tokens] (the prompt -- or
 * prompt + generated after a preemption -- for a request in prefill, else
 * its last token); positions [n]: first position of each request's input;
 * block_tables [n, max_blocks] (-1 padded). */
int rkv_sched_batch(const rkv_scheduler* s, int64_t* request_ids, int32_t* seq_lens,
                    int64_t* input_offsets, int32_t* input_ids, int32_t* positions,
                    int32_t* block_tables, int max_blocks);

/* Scheduler::update (:299-322): appends each request's new token and grows
 * its block table to cover the new length.  RKV_ERR_OOM when the pool is
 * exhausted: the tokens before the failing one are applied, as in the
 * reference's loop, and the failing request keeps its token; the next
 * rkv_sched_schedule pauses it if its table still cannot grow. */
int rkv_sched_update(rkv_scheduler* s, const int64_t* request_ids, const int32_t* tokens, int n);

/* Scheduler stats (:391-438): counts and tokens generated by completed
 * requests.  out[0..4] = pending, running, paused, completed,
 * total_tokens_generated. */
int rkv_sched_stats(const rkv_scheduler* s, int64_t* out5);

/* Generated tokens of a request (running, paused or completed); returns the
 * count, copies at most cap of them, or RKV_ERR_INVALID_ARG for an unknown id. */
int64_t rkv_sched_generated(const rkv_scheduler* s, int64_t request_id, int32_t* out, int64_t cap);

/* The scheduler's block manager (owned by the scheduler; for compaction and
 * table inspection). */
rkv_block_manager* rkv_sched_block_manager(rkv_scheduler* s);

/* Sampler::greedy (continuous_batching.rs:458-462) on host logits: index of
 * the maximum, the LAST one among equal maxima (Iterator::max_by).  Returns
 * -1 for n <= 0 or a NaN (the reference panics on NaN). */
int rkv_sampler_greedy(const float* logits, int n);

#ifdef __cplusplus
}
#endif
#endif /* RUSTRAL_SERVING_H */
