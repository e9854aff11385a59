"""Host-side block manager and continuous-batching scheduler.

Python face of include/rustral_serving.h (the C++ implementation in
csrc/serving.cpp).  Names and behaviour follow rustral's ``PagedCache``
(crates/nn/src/kv_cache.rs:381-432) and ``Scheduler`` / ``Batch`` /
``Sampler`` (crates/nn/src/continuous_batching.rs), with the documented
fixes: allocation appends to a sequence's table, finished and preempted
requests return their blocks, and a batch lists requests by ascending id.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import RKV_ERR_OOM, RkvError, lib

LOW, NORMAL, HIGH, CRITICAL = 0, 1, 2, 3
EOS_TOKEN = 2


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _err(code: int) -> RkvError:
    return RkvError(code, lib().rkv_last_error().decode())


class PagedCache:
    """FIFO block allocator with per-sequence block tables."""

    def __init__(self, block_size: int, num_blocks: int, *, _handle=None, _owner=None):
        if _handle is not None:
            self._h, self._owned, self._owner = _handle, False, _owner
            return
        h = lib().rkv_bm_create(num_blocks, block_size)
        if not h:
            raise _err(-1)
        self._h, self._owned, self._owner = h, True, None

    def __del__(self):
        if getattr(self, "_owned", False) and self._h:
            try:
                lib().rkv_bm_destroy(self._h)
            except Exception:  # interpreter shutdown: the module is torn down
                pass
            self._h = None

    @property
    def block_size(self) -> int:
        return lib().rkv_bm_block_size(self._h)

    @property
    def num_blocks(self) -> int:
        return lib().rkv_bm_num_blocks(self._h)

    def num_free(self) -> int:
        return lib().rkv_bm_num_free(self._h)

    def allocate(self, seq_id: int, num_tokens: int) -> list[int] | None:
        """ceil(num_tokens / block_size) new ids appended to seq_id's table,
        or None when the pool cannot supply them (nothing is taken)."""
        n_max = -(-max(num_tokens, 0) // self.block_size)
        out = np.empty(max(n_max, 1), np.int32)
        n = lib().rkv_bm_allocate(self._h, seq_id, num_tokens, _ptr(out), len(out))
        if n == RKV_ERR_OOM:
            return None
        if n < 0:
            raise _err(n)
        return out[:n].tolist()

    def reserve(self, seq_id: int, num_tokens: int) -> int | None:
        n = lib().rkv_bm_reserve(self._h, seq_id, num_tokens)
        if n == RKV_ERR_OOM:
            return None
        if n < 0:
            raise _err(n)
        return n

    def free(self, seq_id: int) -> int:
        return lib().rkv_bm_free(self._h, seq_id)

    def table(self, seq_id: int) -> list[int]:
        n = lib().rkv_bm_table(self._h, seq_id, None, 0)
        out = np.empty(max(n, 1), np.int32)
        lib().rkv_bm_table(self._h, seq_id, _ptr(out), n)
        return out[:n].tolist()

    def free_list(self) -> list[int]:
        n = lib().rkv_bm_free_list(self._h, None, 0)
        out = np.empty(max(n, 1), np.int32)
        lib().rkv_bm_free_list(self._h, _ptr(out), n)
        return out[:n].tolist()

    def fill_tables(self, seq_ids, max_blocks: int) -> np.ndarray:
        ids = np.ascontiguousarray(seq_ids, dtype=np.int64)
        out = np.empty((len(ids), max_blocks), np.int32)
        rc = lib().rkv_bm_fill_tables(self._h, _ptr(ids), len(ids), _ptr(out), max_blocks)
        if rc:
            raise _err(rc)
        return out

    def plan_compaction(self, max_moves: int) -> np.ndarray:
        """(src, dst) pairs [n, 2] moving the highest live blocks down; the
        tables are rewritten already, the data must follow via copy_blocks."""
        buf = np.empty((max(max_moves, 1), 2), np.int32)
        n = lib().rkv_bm_plan_compaction(self._h, max_moves, _ptr(buf), max_moves)
        if n < 0:
            raise _err(n)
        return buf[:n].copy()

    def plan_migration(self, max_moves: int) -> np.ndarray:
        """Like plan_compaction without the stop at the first free id above
        the source: min(max_moves, live, free) live blocks move, highest
        first, to the lowest free ids."""
        buf = np.empty((max(max_moves, 1), 2), np.int32)
        n = lib().rkv_bm_plan_migration(self._h, max_moves, _ptr(buf), max_moves)
        if n < 0:
            raise _err(n)
        return buf[:n].copy()

    def plan_relocation(self, max_moves: int) -> np.ndarray:
        """The blocks plan_migration moves, into the longest runs of free ids
        (longest first), pairs ascending on both sides."""
        buf = np.empty((max(max_moves, 1), 2), np.int32)
        n = lib().rkv_bm_plan_relocation(self._h, max_moves, _ptr(buf), max_moves)
        if n < 0:
            raise _err(n)
        return buf[:n].copy()


@dataclass
class Batch:
    """One iteration's work (continuous_batching.rs:157-167)."""
    request_ids: list[int]
    input_ids: list[list[int]]
    seq_lens: list[int]
    positions: list[int]
    block_tables: np.ndarray  # int32 [n, max_blocks], -1 padded


class Scheduler:
    def __init__(self, num_blocks: int, block_size: int = 16, max_batch_size: int = 8,
                 max_seq_len: int = 8192):
        h = lib().rkv_sched_create(num_blocks, block_size, max_batch_size, max_seq_len)
        if not h:
            raise _err(-1)
        self._h = h
        self.cache = PagedCache(block_size, num_blocks,
                                _handle=lib().rkv_sched_block_manager(h), _owner=self)

    @classmethod
    def _borrow(cls, handle, owner):
        """A view of a scheduler owned by another object (the serving engine)."""
        s = cls.__new__(cls)
        s._h, s._borrowed, s._owner = handle, True, owner
        s.cache = PagedCache(0, 0, _handle=lib().rkv_sched_block_manager(handle), _owner=s)
        return s

    def __del__(self):
        if getattr(self, "_h", None) and not getattr(self, "_borrowed", False):
            lib().rkv_sched_destroy(self._h)
            self._h = None

    def add_request(self, prompt, max_tokens: int, priority: int = NORMAL) -> int:
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        rid = lib().rkv_sched_add_request(self._h, _ptr(p), len(p), max_tokens, priority)
        if rid < 0:
            raise _err(rid)
        return rid

    def add_priority_request(self, prompt, max_tokens: int, priority: int) -> int:
        return self.add_request(prompt, max_tokens, priority)

    def schedule(self) -> Batch | None:
        n = lib().rkv_sched_schedule(self._h)
        if n < 0:
            raise _err(n)
        if n == 0:
            return None
        nr, nt, mb = C.c_int(), C.c_int64(), C.c_int()
        lib().rkv_sched_batch_dims(self._h, C.byref(nr), C.byref(nt), C.byref(mb))
        nr, nt, mb = nr.value, nt.value, max(mb.value, 1)
        ids = np.empty(nr, np.int64)
        lens = np.empty(nr, np.int32)
        offs = np.empty(nr + 1, np.int64)
        inp = np.empty(max(nt, 1), np.int32)
        pos = np.empty(nr, np.int32)
        tabs = np.empty((nr, mb), np.int32)
        rc = lib().rkv_sched_batch(self._h, _ptr(ids), _ptr(lens), _ptr(offs), _ptr(inp),
                                   _ptr(pos), _ptr(tabs), mb)
        if rc:
            raise _err(rc)
        return Batch(ids.tolist(), [inp[offs[i]:offs[i + 1]].tolist() for i in range(nr)],
                     lens.tolist(), pos.tolist(), tabs)

    def update(self, outputs: dict[int, int]) -> None:
        ids = np.array(list(outputs.keys()), np.int64)
        toks = np.array(list(outputs.values()), np.int32)
        rc = lib().rkv_sched_update(self._h, _ptr(ids), _ptr(toks), len(ids))
        if rc:
            raise _err(rc)

    def stats(self) -> dict:
        out = np.zeros(5, np.int64)
        lib().rkv_sched_stats(self._h, _ptr(out))
        keys = ("pending", "running", "paused", "completed", "total_tokens_generated")
        return dict(zip(keys, out.tolist()))

    def pending_count(self) -> int:
        return self.stats()["pending"]

    def running_count(self) -> int:
        return self.stats()["running"]

    def completed_count(self) -> int:
        return self.stats()["completed"]

    def is_empty(self) -> bool:
        s = self.stats()
        return s["pending"] == 0 and s["running"] == 0 and s["paused"] == 0

    def generated(self, request_id: int) -> list[int]:
        n = lib().rkv_sched_generated(self._h, request_id, None, 0)
        if n < 0:
            raise _err(n)
        out = np.empty(max(n, 1), np.int32)
        lib().rkv_sched_generated(self._h, request_id, _ptr(out), n)
        return out[:n].tolist()


class Sampler:
    @staticmethod
    def greedy(logits) -> int:
        """Index of the maximum, the last one among ties (Iterator::max_by)."""
        a = np.ascontiguousarray(logits, dtype=np.float32)
        r = lib().rkv_sampler_greedy(_ptr(a), len(a))
        if r < 0:
            raise ValueError("greedy sampling of an empty or NaN logit vector")
        return r


__all__ = ["PagedCache", "Scheduler", "Batch", "Sampler", "LOW", "NORMAL", "HIGH", "CRITICAL",
           "EOS_TOKEN"]
