// serving.cpp -- host side of the paged-KV path: the block manager
// (rustral's PagedCache) and the continuous-batching scheduler (Scheduler,
// Batch, Request), behind the C ABI of include/rustral_serving.h.
//
// Host-only C++17; nothing here touches the GPU.  Semantics follow
// crates/nn/src/kv_cache.rs:381-432 and crates/nn/src/continuous_batching.rs,
// with the deviations the header documents (tables append instead of being
// overwritten, completed and preempted requests give their blocks back, the
// batch is ordered by request id).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <deque>
#include <map>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/rustral_kv.h"
#include "../../include/rustral_serving.h"

namespace rkv {
void set_error(const std::string& msg);
void clear_error();
namespace {

int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

// ---- block manager ---------------------------------------------------------

class BlockManager {
 public:
  BlockManager(int64_t num_blocks, int block_size)
      : block_size_(block_size), owner_(num_blocks, -1), pos_(num_blocks, -1) {
    for (int64_t b = 0; b < num_blocks; ++b) free_.push_back((int32_t)b);
  }

  int block_size() const { return block_size_; }
  int64_t num_blocks() const { return (int64_t)owner_.size(); }
  int64_t num_free() const { return (int64_t)free_.size(); }

  int64_t blocks_for(int64_t tokens) const {
    return tokens <= 0 ? 0 : (tokens + block_size_ - 1) / block_size_;
  }

  // Takes n ids from the front of the free list onto seq's table.
  // Returns false (and takes nothing) if fewer than n are free.
  bool take(int64_t seq, int64_t n, std::vector<int32_t>* got) {
    if (n > (int64_t)free_.size()) return false;
    std::vector<int32_t>& t = tables_[seq];
    for (int64_t i = 0; i < n; ++i) {
      const int32_t b = free_.front();
      free_.pop_front();
      owner_[b] = seq;
      pos_[b] = (int64_t)t.size();
      t.push_back(b);
      if (got) got->push_back(b);
    }
    return true;
  }

  int64_t allocate(int64_t seq, int64_t num_tokens, std::vector<int32_t>* got) {
    const int64_t n = blocks_for(num_tokens);
    if (!take(seq, n, got)) return RKV_ERR_OOM;
    return n;
  }

  int64_t reserve(int64_t seq, int64_t num_tokens) {
    const int64_t have = table_len(seq);
    const int64_t want = blocks_for(num_tokens);
    if (want <= have) return 0;
    if (!take(seq, want - have, nullptr)) return RKV_ERR_OOM;
    return want - have;
  }

  int64_t free_seq(int64_t seq) {
    auto it = tables_.find(seq);
    if (it == tables_.end()) return 0;
    const int64_t n = (int64_t)it->second.size();
    for (int32_t b : it->second) {
      owner_[b] = -1;
      pos_[b] = -1;
      free_.push_back(b);
    }
    tables_.erase(it);
    return n;
  }

  const std::vector<int32_t>* table(int64_t seq) const {
    auto it = tables_.find(seq);
    return it == tables_.end() ? nullptr : &it->second;
  }
  int64_t table_len(int64_t seq) const {
    const auto* t = table(seq);
    return t ? (int64_t)t->size() : 0;
  }
  const std::deque<int32_t>& free_list() const { return free_; }

  // Highest live ids move into the lowest free ids: below them only
  // (compaction), or wherever the lowest free ids are (migration).
  int64_t plan_compaction(int64_t max_moves, std::vector<int32_t>* pairs,
                          bool below_only = true) {
    std::vector<int32_t> fr(free_.begin(), free_.end());
    std::sort(fr.begin(), fr.end());
    int64_t moves = 0;
    size_t j = 0;
    std::vector<int32_t> freed;
    // only blocks live before the plan move (a destination of this plan is
    // never moved again, so sources and destinations stay disjoint)
    std::vector<char> dest((size_t)num_blocks(), 0);
    for (int64_t b = num_blocks() - 1; b >= 0 && moves < max_moves && j < fr.size(); --b) {
      if (owner_[b] < 0 || dest[(size_t)b]) continue;
      const int32_t dst = fr[j];
      if (below_only && dst >= b) break;
      ++j;
      dest[(size_t)dst] = 1;
      const int64_t seq = owner_[b], p = pos_[b];
      tables_[seq][p] = dst;
      owner_[dst] = seq;
      pos_[dst] = p;
      owner_[b] = -1;
      pos_[b] = -1;
      pairs->push_back((int32_t)b);
      pairs->push_back(dst);
      freed.push_back((int32_t)b);
      ++moves;
    }
    std::vector<int32_t> rest(fr.begin() + (std::ptrdiff_t)j, fr.end());
    rest.insert(rest.end(), freed.begin(), freed.end());
    std::sort(rest.begin(), rest.end());
    free_.assign(rest.begin(), rest.end());
    return moves;
  }

  // The blocks plan_compaction(.., below_only = false) would move -- the
  // min(max_moves, live, free) highest live ids -- go into the longest runs
  // of consecutive free ids instead of the lowest free ids: runs by length,
  // longest first (lower start on ties), each filled from its low end.  The
  // i-th lowest source goes to the i-th lowest destination, so the pairs
  // come out ascending on both sides and a copy writes whole runs of
  // consecutive blocks.
  int64_t plan_relocation(int64_t max_moves, std::vector<int32_t>* pairs) {
    std::vector<int32_t> fr(free_.begin(), free_.end());
    std::sort(fr.begin(), fr.end());
    std::vector<int32_t> src;
    for (int64_t b = num_blocks() - 1;
         b >= 0 && (int64_t)src.size() < max_moves && src.size() < fr.size(); --b)
      if (owner_[b] >= 0) src.push_back((int32_t)b);
    const size_t n = src.size();
    std::reverse(src.begin(), src.end());
    struct Run { int32_t start, len; };
    std::vector<Run> runs;
    for (size_t i = 0; i < fr.size();) {
      size_t k = i + 1;
      while (k < fr.size() && fr[k] == fr[k - 1] + 1) ++k;
      runs.push_back({fr[i], (int32_t)(k - i)});
      i = k;
    }
    std::stable_sort(runs.begin(), runs.end(),
                     [](const Run& a, const Run& b) { return a.len > b.len; });
    std::vector<int32_t> dst;
    for (const Run& r : runs)
      for (int32_t x = 0; x < r.len && dst.size() < n; ++x) dst.push_back(r.start + x);
    std::sort(dst.begin(), dst.end());
    std::vector<char> taken((size_t)num_blocks(), 0);
    for (size_t i = 0; i < n; ++i) {
      const int32_t b = src[i], d = dst[i];
      const int64_t seq = owner_[b], p = pos_[b];
      tables_[seq][p] = d;
      owner_[d] = seq;
      pos_[d] = p;
      owner_[b] = -1;
      pos_[b] = -1;
      taken[(size_t)d] = 1;
      pairs->push_back(b);
      pairs->push_back(d);
    }
    std::vector<int32_t> rest;
    for (int32_t f : fr)
      if (!taken[(size_t)f]) rest.push_back(f);
    rest.insert(rest.end(), src.begin(), src.end());
    std::sort(rest.begin(), rest.end());
    free_.assign(rest.begin(), rest.end());
    return (int64_t)n;
  }

 private:
  int block_size_;
  std::deque<int32_t> free_;                                  // FIFO
  std::unordered_map<int64_t, std::vector<int32_t>> tables_;  // seq -> ids
  std::vector<int64_t> owner_;                                // block -> seq (-1 = free)
  std::vector<int64_t> pos_;                                  // block -> index in its table
};

// ---- scheduler ---------------------------------------------------------------

using Clock = std::chrono::steady_clock;

enum class State { Waiting, Prefill, Generating, Paused, Completed };

struct Request {
  int64_t id = 0;
  std::vector<int32_t> prompt, generated;
  int max_tokens = 0;
  int priority = RKV_PRIORITY_NORMAL;
  State state = State::Waiting;
  bool recompute = false;  // resumed after preemption: prefill prompt + generated again
  Clock::time_point arrival, last_gen;

  int64_t seq_len() const { return (int64_t)(prompt.size() + generated.size()); }
  bool should_complete() const {
    if ((int64_t)generated.size() >= max_tokens) return true;
    return !generated.empty() && generated.back() == RKV_EOS_TOKEN;
  }
  bool in_prefill() const { return generated.empty() || recompute; }
};

struct BatchRow {
  int64_t id;
  int32_t seq_len;
  int32_t position;
  std::vector<int32_t> input;
  std::vector<int32_t> table;
};

class Scheduler {
 public:
  Scheduler(int64_t num_blocks, int block_size, int max_batch, int max_seq_len)
      : cache_(num_blocks, block_size), max_batch_(max_batch), max_seq_len_(max_seq_len) {}

  BlockManager& cache() { return cache_; }

  int64_t add(const int32_t* prompt, int n, int max_tokens, int priority) {
    Request r;
    r.id = next_id_++;
    r.prompt.assign(prompt, prompt + n);
    r.max_tokens = max_tokens;
    r.priority = priority;
    r.arrival = r.last_gen = Clock::now();
    pending_.push_back(std::move(r));
    return pending_.back().id;
  }

  int schedule() {
    // 1. retire finished requests
    for (auto it = running_.begin(); it != running_.end();) {
      if (it->second.should_complete()) {
        cache_.free_seq(it->first);
        it->second.state = State::Completed;
        completed_.push_back(std::move(it->second));
        it = running_.erase(it);
      } else {
        ++it;
      }
    }
    // 1b. a running request whose last update found no free block (its table
    // no longer covers its sequence) retries the reservation; if the pool is
    // still full it is paused like a preempted request and later resumes by
    // recompute -- the "should preempt" of the reference's out-of-memory
    // branch (continuous_batching.rs:313-315).  Ascending id.
    for (auto it = running_.begin(); it != running_.end();) {
      Request& r = it->second;
      if (cache_.reserve(r.id, r.seq_len()) >= 0) {
        ++it;
        continue;
      }
      cache_.free_seq(r.id);
      r.state = State::Paused;
      paused_.push_back(std::move(r));
      it = running_.erase(it);
    }
    // 2. resume paused requests (in pause order) while there is room
    while (!paused_.empty() && (int)running_.size() < max_batch_) {
      Request& r = paused_.front();
      if (cache_.reserve(r.id, r.seq_len()) < 0) break;
      r.state = State::Prefill;
      r.recompute = !r.generated.empty();
      running_.emplace(r.id, std::move(r));
      paused_.pop_front();
    }
    // 3. admit pending requests
    while ((int)running_.size() < max_batch_ && !pending_.empty()) {
      Request& r = pending_.front();
      if (cache_.allocate(r.id, (int64_t)r.prompt.size(), nullptr) < 0) break;
      r.state = State::Prefill;
      running_.emplace(r.id, std::move(r));
      pending_.pop_front();
    }
    // 4. preempt one Low-priority request under pressure (lowest id first)
    const float pressure = max_batch_ > 0 ? (float)running_.size() / (float)max_batch_ : 0.0f;
    if (pressure > kPreemptionThreshold) {
      for (auto it = running_.begin(); it != running_.end(); ++it) {
        if (it->second.priority == RKV_PRIORITY_LOW) {
          cache_.free_seq(it->first);
          it->second.state = State::Paused;
          paused_.push_back(std::move(it->second));
          running_.erase(it);
          break;
        }
      }
    }
    // 5. the batch, ascending id (std::map order)
    batch_.clear();
    for (auto& kv : running_) {
      Request& r = kv.second;
      BatchRow row;
      row.id = r.id;
      row.seq_len = (int32_t)r.seq_len();
      if (r.in_prefill()) {
        row.input = r.prompt;
        if (r.recompute) row.input.insert(row.input.end(), r.generated.begin(), r.generated.end());
        row.position = 0;
      } else {
        row.input.push_back(r.generated.back());
        row.position = row.seq_len - 1;
      }
      if (const auto* t = cache_.table(r.id)) row.table = *t;
      batch_.push_back(std::move(row));
    }
    return (int)batch_.size();
  }

  const std::vector<BatchRow>& batch() const { return batch_; }

  int update(const int64_t* ids, const int32_t* tokens, int n) {
    for (int i = 0; i < n; ++i) {
      auto it = running_.find(ids[i]);
      if (it == running_.end()) continue;
      Request& r = it->second;
      r.generated.push_back(tokens[i]);
      r.last_gen = Clock::now();
      r.recompute = false;
      r.state = State::Generating;
      if (cache_.reserve(r.id, r.seq_len()) < 0)
        return fail(RKV_ERR_OOM, "KV cache out of memory");
    }
    return RKV_OK;
  }

  void stats(int64_t* out) const {
    int64_t toks = 0;
    for (const auto& r : completed_) toks += (int64_t)r.generated.size();
    out[0] = (int64_t)pending_.size();
    out[1] = (int64_t)running_.size();
    out[2] = (int64_t)paused_.size();
    out[3] = (int64_t)completed_.size();
    out[4] = toks;
  }

  const Request* find(int64_t id) const {
    auto it = running_.find(id);
    if (it != running_.end()) return &it->second;
    for (const auto& r : paused_)
      if (r.id == id) return &r;
    for (const auto& r : completed_)
      if (r.id == id) return &r;
    for (const auto& r : pending_)
      if (r.id == id) return &r;
    return nullptr;
  }

  int max_seq_len() const { return max_seq_len_; }

 private:
  static constexpr float kPreemptionThreshold = 0.5f;
  BlockManager cache_;
  int max_batch_, max_seq_len_;
  int64_t next_id_ = 0;
  std::deque<Request> pending_, paused_;
  std::map<int64_t, Request> running_;
  std::vector<Request> completed_;
  std::vector<BatchRow> batch_;
};

}  // namespace
}  // namespace rkv

struct rkv_block_manager {
  rkv::BlockManager* bm;
  bool owned;
};
struct rkv_scheduler {
  rkv::Scheduler s;
  rkv_block_manager view;
};

using rkv::fail;

extern "C" rkv_block_manager* rkv_bm_create(int64_t num_blocks, int block_size) {
  rkv::clear_error();
  if (num_blocks < 0 || num_blocks > INT32_MAX || block_size <= 0) {
    rkv::set_error("rkv_bm_create: num_blocks must be in [0, 2^31) and block_size > 0");
    return nullptr;
  }
  auto* bm = new (std::nothrow) rkv::BlockManager(num_blocks, block_size);
  if (!bm) return nullptr;
  return new rkv_block_manager{bm, true};
}

extern "C" void rkv_bm_destroy(rkv_block_manager* bm) {
  if (!bm || !bm->owned) return;
  delete bm->bm;
  delete bm;
}

extern "C" int64_t rkv_bm_allocate(rkv_block_manager* bm, int64_t seq_id, int64_t num_tokens,
                                   int32_t* out_ids, int64_t cap) {
  rkv::clear_error();
  if (!bm || num_tokens < 0) return fail(RKV_ERR_INVALID_ARG, "rkv_bm_allocate: bad argument");
  std::vector<int32_t> got;
  const int64_t n = bm->bm->allocate(seq_id, num_tokens, &got);
  if (n < 0) return fail(RKV_ERR_OOM, "KV cache out of memory");
  if (out_ids)
    for (int64_t i = 0; i < n && i < cap; ++i) out_ids[i] = got[(size_t)i];
  return n;
}

extern "C" int64_t rkv_bm_reserve(rkv_block_manager* bm, int64_t seq_id, int64_t num_tokens) {
  rkv::clear_error();
  if (!bm || num_tokens < 0) return fail(RKV_ERR_INVALID_ARG, "rkv_bm_reserve: bad argument");
  const int64_t n = bm->bm->reserve(seq_id, num_tokens);
  if (n < 0) return fail(RKV_ERR_OOM, "KV cache out of memory");
  return n;
}

extern "C" int64_t rkv_bm_free(rkv_block_manager* bm, int64_t seq_id) {
  return bm ? bm->bm->free_seq(seq_id) : 0;
}

extern "C" int64_t rkv_bm_num_free(const rkv_block_manager* bm) {
  return bm ? bm->bm->num_free() : 0;
}
extern "C" int64_t rkv_bm_num_blocks(const rkv_block_manager* bm) {
  return bm ? bm->bm->num_blocks() : 0;
}
extern "C" int rkv_bm_block_size(const rkv_block_manager* bm) {
  return bm ? bm->bm->block_size() : 0;
}

extern "C" int64_t rkv_bm_table(const rkv_block_manager* bm, int64_t seq_id, int32_t* out,
                                int64_t cap) {
  if (!bm) return 0;
  const auto* t = bm->bm->table(seq_id);
  if (!t) return 0;
  if (out)
    for (int64_t i = 0; i < (int64_t)t->size() && i < cap; ++i) out[i] = (*t)[(size_t)i];
  return (int64_t)t->size();
}

extern "C" int64_t rkv_bm_free_list(const rkv_block_manager* bm, int32_t* out, int64_t cap) {
  if (!bm) return 0;
  const auto& f = bm->bm->free_list();
  if (out) {
    int64_t i = 0;
    for (auto it = f.begin(); it != f.end() && i < cap; ++it) out[i++] = *it;
  }
  return (int64_t)f.size();
}

extern "C" int rkv_bm_fill_tables(const rkv_block_manager* bm, const int64_t* seq_ids,
                                  int n_seqs, int32_t* tables, int max_blocks) {
  rkv::clear_error();
  if (!bm || n_seqs < 0 || max_blocks < 0 || (n_seqs > 0 && (!seq_ids || !tables)))
    return fail(RKV_ERR_INVALID_ARG, "rkv_bm_fill_tables: bad argument");
  for (int i = 0; i < n_seqs; ++i) {
    const auto* t = bm->bm->table(seq_ids[i]);
    const int64_t n = t ? (int64_t)t->size() : 0;
    if (n > max_blocks)
      return fail(RKV_ERR_INVALID_ARG, "rkv_bm_fill_tables: a table is longer than max_blocks");
    int32_t* row = tables + (int64_t)i * max_blocks;
    for (int64_t j = 0; j < max_blocks; ++j) row[j] = j < n ? (*t)[(size_t)j] : -1;
  }
  return RKV_OK;
}

extern "C" int64_t rkv_bm_plan_compaction(rkv_block_manager* bm, int64_t max_moves,
                                          int32_t* pairs, int64_t cap_pairs) {
  rkv::clear_error();
  if (!bm || max_moves < 0 || cap_pairs < 0 || (max_moves > 0 && !pairs))
    return fail(RKV_ERR_INVALID_ARG, "rkv_bm_plan_compaction: bad argument");
  std::vector<int32_t> p;
  const int64_t n = bm->bm->plan_compaction(std::min(max_moves, cap_pairs), &p);
  std::memcpy(pairs, p.data(), p.size() * sizeof(int32_t));
  return n;
}

extern "C" int64_t rkv_bm_plan_migration(rkv_block_manager* bm, int64_t max_moves,
                                         int32_t* pairs, int64_t cap_pairs) {
  rkv::clear_error();
  if (!bm || max_moves < 0 || cap_pairs < 0 || (max_moves > 0 && !pairs))
    return fail(RKV_ERR_INVALID_ARG, "rkv_bm_plan_migration: bad argument");
  std::vector<int32_t> p;
  const int64_t n = bm->bm->plan_compaction(std::min(max_moves, cap_pairs), &p, false);
  std::memcpy(pairs, p.data(), p.size() * sizeof(int32_t));
  return n;
}

extern "C" int64_t rkv_bm_plan_relocation(rkv_block_manager* bm, int64_t max_moves,
                                          int32_t* pairs, int64_t cap_pairs) {
  rkv::clear_error();
  if (!bm || max_moves < 0 || cap_pairs < 0 || (max_moves > 0 && !pairs))
    return fail(RKV_ERR_INVALID_ARG, "rkv_bm_plan_relocation: bad argument");
  std::vector<int32_t> p;
  const int64_t n = bm->bm->plan_relocation(std::min(max_moves, cap_pairs), &p);
  std::memcpy(pairs, p.data(), p.size() * sizeof(int32_t));
  return n;
}

extern "C" rkv_scheduler* rkv_sched_create(int64_t num_blocks, int block_size,
                                           int max_batch_size, int max_seq_len) {
  rkv::clear_error();
  if (num_blocks < 0 || num_blocks > INT32_MAX || block_size <= 0 || max_batch_size <= 0 ||
      max_seq_len <= 0) {
    rkv::set_error("rkv_sched_create: bad argument");
    return nullptr;
  }
  auto* s = new (std::nothrow)
      rkv_scheduler{rkv::Scheduler(num_blocks, block_size, max_batch_size, max_seq_len), {}};
  if (!s) return nullptr;
  s->view = rkv_block_manager{&s->s.cache(), false};
  return s;
}

extern "C" void rkv_sched_destroy(rkv_scheduler* s) { delete s; }

extern "C" int64_t rkv_sched_add_request(rkv_scheduler* s, const int32_t* prompt, int n_prompt,
                                         int max_tokens, int priority) {
  rkv::clear_error();
  if (!s || n_prompt < 0 || (n_prompt > 0 && !prompt) || max_tokens < 0)
    return fail(RKV_ERR_INVALID_ARG, "rkv_sched_add_request: bad argument");
  if (priority < RKV_PRIORITY_LOW || priority > RKV_PRIORITY_CRITICAL)
    return fail(RKV_ERR_INVALID_ARG, "rkv_sched_add_request: priority must be 0..3");
  if ((int64_t)n_prompt + max_tokens > s->s.max_seq_len())
    return fail(RKV_ERR_INVALID_ARG, "rkv_sched_add_request: prompt + max_tokens > max_seq_len");
  return s->s.add(prompt, n_prompt, max_tokens, priority);
}

extern "C" int rkv_sched_schedule(rkv_scheduler* s) {
  rkv::clear_error();
  if (!s) return fail(RKV_ERR_INVALID_ARG, "rkv_sched_schedule: null handle");
  return s->s.schedule();
}

extern "C" int rkv_sched_batch_dims(const rkv_scheduler* s, int* n_requests,
                                    int64_t* n_input_tokens, int* max_blocks) {
  if (!s) return fail(RKV_ERR_INVALID_ARG, "rkv_sched_batch_dims: null handle");
  int64_t toks = 0;
  int mb = 0;
  for (const auto& r : s->s.batch()) {
    toks += (int64_t)r.input.size();
    mb = std::max(mb, (int)r.table.size());
  }
  if (n_requests) *n_requests = (int)s->s.batch().size();
  if (n_input_tokens) *n_input_tokens = toks;
  if (max_blocks) *max_blocks = mb;
  return RKV_OK;
}

extern "C" int rkv_sched_batch(const rkv_scheduler* s, int64_t* request_ids, int32_t* seq_lens,
                               int64_t* input_offsets, int32_t* input_ids, int32_t* positions,
                               int32_t* block_tables, int max_blocks) {
  rkv::clear_error();
  if (!s) return fail(RKV_ERR_INVALID_ARG, "rkv_sched_batch: null handle");
  const auto& b = s->s.batch();
  if (block_tables) {
    for (const auto& r : b)
      if ((int)r.table.size() > max_blocks)
        return fail(RKV_ERR_INVALID_ARG, "rkv_sched_batch: max_blocks below the longest table");
  }
  int64_t off = 0;
  for (size_t i = 0; i < b.size(); ++i) {
    const auto& r = b[i];
    if (request_ids) request_ids[i] = r.id;
    if (seq_lens) seq_lens[i] = r.seq_len;
    if (positions) positions[i] = r.position;
    if (input_offsets) input_offsets[i] = off;
    if (input_ids) std::memcpy(input_ids + off, r.input.data(), r.input.size() * sizeof(int32_t));
    off += (int64_t)r.input.size();
    if (block_tables) {
      int32_t* row = block_tables + (int64_t)i * max_blocks;
      for (int j = 0; j < max_blocks; ++j) row[j] = j < (int)r.table.size() ? r.table[(size_t)j] : -1;
    }
  }
  if (input_offsets) input_offsets[b.size()] = off;
  return RKV_OK;
}

extern "C" int rkv_sched_update(rkv_scheduler* s, const int64_t* request_ids,
                                const int32_t* tokens, int n) {
  rkv::clear_error();
  if (!s || n < 0 || (n > 0 && (!request_ids || !tokens)))
    return fail(RKV_ERR_INVALID_ARG, "rkv_sched_update: bad argument");
  return s->s.update(request_ids, tokens, n);
}

extern "C" int rkv_sched_stats(const rkv_scheduler* s, int64_t* out5) {
  if (!s || !out5) return fail(RKV_ERR_INVALID_ARG, "rkv_sched_stats: bad argument");
  s->s.stats(out5);
  return RKV_OK;
}

extern "C" int64_t rkv_sched_generated(const rkv_scheduler* s, int64_t request_id, int32_t* out,
                                       int64_t cap) {
  if (!s) return fail(RKV_ERR_INVALID_ARG, "rkv_sched_generated: null handle");
  const auto* r = s->s.find(request_id);
  if (!r) return fail(RKV_ERR_INVALID_ARG, "rkv_sched_generated: unknown request id");
  if (out)
    for (int64_t i = 0; i < (int64_t)r->generated.size() && i < cap; ++i)
      out[i] = r->generated[(size_t)i];
  return (int64_t)r->generated.size();
}

extern "C" rkv_block_manager* rkv_sched_block_manager(rkv_scheduler* s) {
  return s ? &s->view : nullptr;
}

extern "C" int rkv_sampler_greedy(const float* logits, int n) {
  if (!logits || n <= 0) return -1;
  int best = 0;
  for (int i = 0; i < n; ++i) {
    if (std::isnan(logits[i])) return -1;
    if (logits[i] >= logits[best]) best = i;  // ">=": the last maximum wins, like max_by
  }
  return best;
}
