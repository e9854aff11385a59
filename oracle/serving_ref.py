"""Pure-Python restatement of rustral's PagedCache and Scheduler.

TEST INFRASTRUCTURE ONLY: tests/ drive it side by side with the C++ block
manager and scheduler (rustral_amd/csrc/serving.cpp) on the same operation
sequences.  The product never imports it.

Follows crates/nn/src/kv_cache.rs:381-432 (PagedCache) and
crates/nn/src/continuous_batching.rs:195-389 (Scheduler), plus the fixes the
C ABI documents (include/rustral_serving.h):
  * allocate appends to a sequence's table (the reference overwrites it,
    kv_cache.rs:422, leaking the earlier blocks);
  * completed requests free their blocks (the reference keeps them,
    continuous_batching.rs:253-260);
  * resumed requests re-allocate blocks for prompt + generated and recompute
    (the reference resumes them with an empty table, :349-363);
  * the batch is in ascending request id (HashMap order, :274);
  * the preempted Low-priority request is the lowest id among them
    (min_by_key over equal keys in HashMap order, :371-377).
Written as plain lists and dicts, independently of the C++ code.
"""
from __future__ import annotations


class PagedCacheRef:
    def __init__(self, block_size: int, num_blocks: int):
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.free_blocks = list(range(num_blocks))       # kv_cache.rs:407
        self.block_tables: dict[int, list[int]] = {}

    def blocks_for(self, tokens: int) -> int:
        return (tokens + self.block_size - 1) // self.block_size if tokens > 0 else 0

    def allocate(self, seq_id: int, num_tokens: int):
        n = self.blocks_for(num_tokens)                   # kv_cache.rs:414
        if len(self.free_blocks) < n:                     # :416-418
            return None
        got = self.free_blocks[:n]                        # drain(0..n), :420
        del self.free_blocks[:n]
        self.block_tables.setdefault(seq_id, []).extend(got)
        return got

    def reserve(self, seq_id: int, num_tokens: int):
        have = len(self.block_tables.get(seq_id, []))
        want = self.blocks_for(num_tokens)
        if want <= have:
            return 0
        got = self.allocate(seq_id, (want - have) * self.block_size)
        return None if got is None else len(got)

    def free(self, seq_id: int) -> int:
        blocks = self.block_tables.pop(seq_id, None)     # :428
        if blocks is None:
            return 0
        self.free_blocks.extend(blocks)                   # :429
        return len(blocks)

    def table(self, seq_id: int) -> list[int]:
        return list(self.block_tables.get(seq_id, []))

    def plan_migration(self, max_moves: int):
        return self.plan_compaction(max_moves, below_only=False)

    def plan_relocation(self, max_moves: int):
        """plan_migration's sources into the longest free runs (longest first,
        lower start on ties), i-th lowest source to i-th lowest destination."""
        owner = {}
        for s, t in self.block_tables.items():
            for i, b in enumerate(t):
                owner[b] = (s, i)
        free = sorted(self.free_blocks)
        n = min(max_moves, len(owner), len(free))
        src = sorted(sorted(owner, reverse=True)[:n])
        runs = []
        for f in free:
            if runs and runs[-1][0] + runs[-1][1] == f:
                runs[-1][1] += 1
            else:
                runs.append([f, 1])
        runs.sort(key=lambda r: (-r[1], r[0]))
        dst = sorted([r[0] + x for r in runs for x in range(r[1])][:n])
        for b, d in zip(src, dst):
            s, i = owner[b]
            self.block_tables[s][i] = d
        taken = set(dst)
        self.free_blocks = sorted([f for f in free if f not in taken] + src)
        return list(zip(src, dst))

    def plan_compaction(self, max_moves: int, below_only: bool = True):
        owner = {}
        for s, t in self.block_tables.items():
            for i, b in enumerate(t):
                owner[b] = (s, i)
        live = sorted(owner, reverse=True)
        free = sorted(self.free_blocks)
        pairs, j = [], 0
        for b in live:
            if len(pairs) >= max_moves or j >= len(free) or (below_only and free[j] >= b):
                break
            s, i = owner[b]
            self.block_tables[s][i] = free[j]
            pairs.append((b, free[j]))
            j += 1
        self.free_blocks = sorted(free[j:] + [p[0] for p in pairs])
        return pairs


class RequestRef:
    def __init__(self, rid, prompt, max_tokens, priority):
        self.id, self.prompt, self.generated = rid, list(prompt), []
        self.max_tokens, self.priority = max_tokens, priority
        self.recompute = False

    def seq_len(self):
        return len(self.prompt) + len(self.generated)

    def should_complete(self):                             # continuous_batching.rs:118-131
        if len(self.generated) >= self.max_tokens:
            return True
        return bool(self.generated) and self.generated[-1] == 2


class SchedulerRef:
    def __init__(self, num_blocks, block_size, max_batch_size, max_seq_len):
        self.cache = PagedCacheRef(block_size, num_blocks)
        self.max_batch, self.max_seq_len = max_batch_size, max_seq_len
        self.pending, self.running, self.paused, self.completed = [], {}, [], []
        self.next_id = 0
        self.threshold = 0.5                               # :217

    def add_request(self, prompt, max_tokens, priority=1):
        rid = self.next_id
        self.next_id += 1
        self.pending.append(RequestRef(rid, prompt, max_tokens, priority))
        return rid

    def schedule(self):
        for rid in sorted(self.running):                   # 1. retire
            if self.running[rid].should_complete():
                self.cache.free(rid)
                self.completed.append(self.running.pop(rid))
        for rid in sorted(self.running):                   # 1b. starved by an OOM update
            r = self.running[rid]
            if self.cache.reserve(rid, r.seq_len()) is None:   # :313-315 "should preempt"
                self.cache.free(rid)
                self.paused.append(self.running.pop(rid))
        while self.paused and len(self.running) < self.max_batch:  # 2. resume
            r = self.paused[0]
            if self.cache.reserve(r.id, r.seq_len()) is None:
                break
            r.recompute = bool(r.generated)
            self.running[r.id] = self.paused.pop(0)
        while len(self.running) < self.max_batch and self.pending:  # 3. admit
            r = self.pending[0]
            if self.cache.allocate(r.id, len(r.prompt)) is None:
                break
            self.running[r.id] = self.pending.pop(0)
        if self.running and len(self.running) / self.max_batch > self.threshold:  # 4. preempt
            lows = [rid for rid in sorted(self.running) if self.running[rid].priority == 0]
            if lows:
                r = self.running.pop(lows[0])
                self.cache.free(r.id)
                self.paused.append(r)
        if not self.running:
            return None
        rows = []
        for rid in sorted(self.running):                   # 5. batch
            r = self.running[rid]
            if not r.generated or r.recompute:
                inp, pos = r.prompt + (r.generated if r.recompute else []), 0
            else:
                inp, pos = [r.generated[-1]], r.seq_len() - 1
            rows.append((rid, inp, r.seq_len(), pos, self.cache.table(rid)))
        return rows

    def update(self, outputs: dict):
        for rid, tok in outputs.items():
            r = self.running.get(rid)
            if r is None:
                continue
            r.generated.append(tok)
            r.recompute = False
            if self.cache.reserve(rid, r.seq_len()) is None:
                return False
        return True

    def stats(self):
        return dict(pending=len(self.pending), running=len(self.running), paused=len(self.paused),
                    completed=len(self.completed),
                    total_tokens_generated=sum(len(r.generated) for r in self.completed))


def greedy_ref(logits) -> int:
    """Sampler::greedy (continuous_batching.rs:458-462): max_by keeps the last maximum."""
    best = 0
    for i, v in enumerate(logits):
        if v >= logits[best]:
            best = i
    return best
