"""Host-side block manager and scheduler (CPU only).

Three kinds of checks:
  * the reference's own unit tests for PagedCache / Scheduler / Sampler
    (crates/nn/src/kv_cache.rs:538-550, :662-669;
    crates/nn/src/continuous_batching.rs:546-717), restated;
  * differential runs against the pure-Python restatement in
    oracle/serving_ref.py on random operation sequences;
  * invariants: every block is either free or in exactly one table, tables
    cover their sequences, compaction keeps the data a gather would see.
"""
import random

import numpy as np
import pytest

from oracle.serving_ref import PagedCacheRef, SchedulerRef, greedy_ref
from rustral_amd.serving import LOW, NORMAL, HIGH, PagedCache, Sampler, Scheduler


# ---- the reference's tests ---------------------------------------------------

def test_paged_cache_reference_case():
    # kv_cache.rs:538-550: 100 tokens -> ceil(100/16) = 7 blocks; free returns all
    c = PagedCache(16, 100)
    blocks = c.allocate(0, 100)
    assert blocks is not None and len(blocks) == 7
    c.free(0)
    assert c.num_free() == 100


def test_paged_cache_oom_reference_case():
    # kv_cache.rs:662-669: 7 blocks wanted, 2 exist -> None, nothing taken
    c = PagedCache(16, 2)
    assert c.allocate(0, 100) is None
    assert c.num_free() == 2


def test_fifo_order_and_append_fix():
    c = PagedCache(16, 10)
    assert c.allocate(5, 20) == [0, 1]            # drain(0..n) from the front
    assert c.allocate(6, 1) == [2]
    assert c.allocate(5, 16) == [3]               # appended, not overwritten
    assert c.table(5) == [0, 1, 3]
    assert c.free(5) == 3                         # every block of the sequence comes back
    assert c.free_list() == [4, 5, 6, 7, 8, 9, 0, 1, 3]   # to the back, table order
    assert c.free(42) == 0


def test_zero_tokens_allocate_nothing():
    c = PagedCache(16, 4)
    assert c.allocate(1, 0) == []
    assert c.num_free() == 4


def test_sampler_greedy_reference_fixture_and_ties():
    # continuous_batching.rs:585-589
    assert Sampler.greedy([0.1, 0.5, 0.3, 0.9, 0.2]) == 3
    assert Sampler.greedy([1.0, 3.0, 3.0, 0.0]) == 2      # max_by: last maximum
    assert Sampler.greedy([-1.0]) == 0
    with pytest.raises(ValueError):
        Sampler.greedy([0.0, float("nan")])


def test_scheduler_counts_reference_cases():
    # continuous_batching.rs:591-611, :629-638
    s = Scheduler(100, 16, 8, 8192)
    assert s.stats()["pending"] == 0 and s.stats()["running"] == 0
    s.add_request([1, 2, 3], 100)
    s.add_request([4, 5], 50)
    assert s.pending_count() == 2 and not s.is_empty()
    assert s.add_priority_request([1, 2, 3], 100, HIGH) == 2


def test_scheduler_schedule_and_update_reference_case():
    # continuous_batching.rs:641-658
    s = Scheduler(100, 16, 8, 8192)
    rid = s.add_request([1, 2, 3], 5)
    b = s.schedule()
    assert b is not None and rid in b.request_ids
    assert b.input_ids == [[1, 2, 3]] and b.seq_lens == [3] and b.positions == [0]
    s.update({rid: 10})
    assert s.running_count() == 1
    b = s.schedule()
    assert b.input_ids == [[10]] and b.seq_lens == [4] and b.positions == [3]


def test_scheduler_completion_reference_case():
    # continuous_batching.rs:661-679 and :697-711
    s = Scheduler(100, 16, 8, 8192)
    rid = s.add_request([1, 2], 1)
    assert len(s.schedule().request_ids) == 1
    s.update({rid: 1})
    assert s.schedule() is None
    st = s.stats()
    assert (st["completed"], st["running"], st["pending"]) == (1, 0, 0)
    assert st["total_tokens_generated"] == 1
    assert s.cache.num_free() == 100            # finished requests return their blocks


def test_eos_stops_a_request():
    # Request::should_complete: token 2 is EOS (continuous_batching.rs:124-129)
    s = Scheduler(100, 16, 8, 8192)
    rid = s.add_request([7, 7], 10)
    s.schedule()
    s.update({rid: 2})
    assert s.schedule() is None and s.generated(rid) == [2]


def test_serving_loop_runs_to_completion():
    # continuous_batching.rs:697-717 with real block accounting
    s = Scheduler(100, 16, 8, 8192)
    ids = [s.add_request([1, 2, 3], 2), s.add_request([4] * 40, 3)]
    steps = 0
    while not s.is_empty():
        b = s.schedule()
        if b is None:
            break
        s.update({rid: 1 for rid in b.request_ids})
        steps += 1
    assert steps == 3 and s.completed_count() == 2
    assert [s.generated(i) for i in ids] == [[1, 1], [1, 1, 1]]
    assert s.cache.num_free() == 100


def test_update_reports_oom():
    s = Scheduler(1, 16, 8, 8192)
    rid = s.add_request([3] * 16, 5)
    s.schedule()
    with pytest.raises(RuntimeError, match="out of memory"):
        s.update({rid: 4})                       # 17 tokens need a second block


def test_add_request_rejects_too_long():
    s = Scheduler(10, 16, 4, 64)
    with pytest.raises(RuntimeError):
        s.add_request([1] * 60, 10)


# ---- differential against oracle/serving_ref.py -------------------------------

def _check_tables(cache_c: PagedCache, ref: PagedCacheRef):
    assert cache_c.free_list() == ref.free_blocks
    owned = set(ref.free_blocks)
    for sid, t in ref.block_tables.items():
        assert cache_c.table(sid) == t
        assert not owned & set(t)
        owned |= set(t)
    assert owned == set(range(ref.num_blocks))


@pytest.mark.parametrize("seed", range(6))
def test_block_manager_matches_restatement(seed):
    rng = random.Random(seed)
    nb, bs = rng.choice([(64, 16), (300, 16), (50, 8)])
    c, r = PagedCache(bs, nb), PagedCacheRef(bs, nb)
    for _ in range(400):
        op = rng.random()
        sid = rng.randrange(12)
        if op < 0.45:
            n = rng.randrange(0, 70)
            assert c.allocate(sid, n) == r.allocate(sid, n)
        elif op < 0.6:
            n = rng.randrange(0, 200)
            assert c.reserve(sid, n) == r.reserve(sid, n)
        elif op < 0.85:
            assert c.free(sid) == r.free(sid)
        elif op < 0.93:
            m = rng.randrange(0, 20)
            got = c.plan_compaction(m)
            want = r.plan_compaction(m)
            assert [tuple(p) for p in got.tolist()] == want
            assert len(set(got[:, 0].tolist()) & set(got[:, 1].tolist())) == 0
        elif op < 0.965:
            m = rng.randrange(0, 20)
            got = c.plan_migration(m)
            want = r.plan_migration(m)
            assert [tuple(p) for p in got.tolist()] == want
            assert len(set(got[:, 0].tolist()) & set(got[:, 1].tolist())) == 0
        else:
            m = rng.randrange(0, 20)
            got = c.plan_relocation(m)
            want = r.plan_relocation(m)
            assert [tuple(p) for p in got.tolist()] == want
            assert len(set(got[:, 0].tolist()) & set(got[:, 1].tolist())) == 0
        _check_tables(c, r)


@pytest.mark.parametrize("seed", range(5))
def test_scheduler_matches_restatement(seed):
    rng = random.Random(100 + seed)
    nb, mb = rng.choice([(40, 4), (200, 8), (30, 3)])
    s, ref = Scheduler(nb, 16, mb, 512), SchedulerRef(nb, 16, mb, 512)
    for step in range(120):
        if rng.random() < 0.4:
            prompt = [rng.randrange(1000) for _ in range(rng.randrange(1, 60))]
            mt = rng.randrange(1, 30)
            pr = rng.choice([LOW, NORMAL, NORMAL, HIGH])
            assert s.add_request(prompt, mt, pr) == ref.add_request(prompt, mt, pr)
        b = s.schedule()
        rows = ref.schedule()
        if rows is None:
            assert b is None
            continue
        assert b.request_ids == [x[0] for x in rows]
        assert b.input_ids == [x[1] for x in rows]
        assert b.seq_lens == [x[2] for x in rows]
        assert b.positions == [x[3] for x in rows]
        for i, x in enumerate(rows):
            t = b.block_tables[i]
            assert t[t >= 0].tolist() == x[4]
            assert len(x[4]) * 16 >= x[2]            # the table covers the sequence
        out = {rid: rng.choice([1, 3, 5, 2 if rng.random() < 0.05 else 4]) for rid in b.request_ids}
        ok_ref = ref.update(out)
        try:
            s.update(out)
            ok = True
        except RuntimeError:
            ok = False
        assert ok == ok_ref
        assert s.stats() == ref.stats()
        # after an out-of-memory update the run goes on: the next schedule
        # pauses the starved request (both sides), so tables keep covering
        # their sequences


def test_update_oom_then_schedule_pauses_the_starved_request():
    """An update that finds no free block keeps the token (the reference adds
    it before allocating, continuous_batching.rs:301-316); the next schedule
    must not hand out a row whose table is too short: the request is paused
    and resumes by recompute once blocks are free."""
    s, ref = Scheduler(3, 16, 4, 512), SchedulerRef(3, 16, 4, 512)
    a = s.add_request([5] * 16, 8)
    b = s.add_request([6] * 31, 8)
    assert ref.add_request([5] * 16, 8) == a and ref.add_request([6] * 31, 8) == b
    s.schedule(), ref.schedule()                   # a: 1 block, b: 2 blocks, pool empty
    with pytest.raises(RuntimeError, match="out of memory"):
        s.update({a: 7, b: 7})                     # a needs a second block
    assert ref.update({a: 7, b: 7}) is False
    bt = s.schedule()
    rows = ref.schedule()
    assert bt.request_ids == [x[0] for x in rows] == [b]
    for i, x in enumerate(rows):
        t = bt.block_tables[i]
        assert t[t >= 0].tolist() == x[4] and len(x[4]) * 16 >= x[2]
    assert s.stats() == ref.stats() and s.stats()["paused"] == 1
    # b finishes; a resumes by recomputing prompt + its kept token
    while True:
        out = {rid: 4 for rid in bt.request_ids}
        s.update(out), ref.update(out)
        bt, rows = s.schedule(), ref.schedule()
        if bt is None or a in bt.request_ids:
            break
    assert rows is not None and bt.request_ids == [x[0] for x in rows]
    i = bt.request_ids.index(a)
    assert bt.input_ids[i] == [5] * 16 + [7] == rows[i][1] and bt.positions[i] == 0


# ---- compaction moves data the way copy_blocks does ----------------------------

def test_compaction_plan_preserves_gathered_data():
    rng = np.random.default_rng(3)
    nb, bs = 64, 16
    c = PagedCache(bs, nb)
    for sid in range(10):
        c.allocate(sid, int(rng.integers(1, 100)))
    for sid in (1, 4, 7):
        c.free(sid)
    pool = rng.standard_normal((nb, 2, bs, 8)).astype(np.float32)
    live = [s for s in range(10) if c.table(s)]
    before = {s: pool[c.table(s)].copy() for s in live}
    pairs = c.plan_compaction(1000)
    assert len(pairs) > 0
    src, dst = pairs[:, 0], pairs[:, 1]
    assert (dst < src).all() and not set(src.tolist()) & set(dst.tolist())
    pool[dst] = pool[src]                      # what rkv_copy_blocks does on the device
    for s in live:
        np.testing.assert_array_equal(pool[c.table(s)], before[s])
    n_live = sum(len(c.table(s)) for s in live)
    assert sorted(b for s in live for b in c.table(s)) == list(range(n_live))  # dense
    assert c.free_list() == list(range(n_live, nb))


def test_greedy_ref_matches_library_on_random_vectors():
    rng = np.random.default_rng(0)
    for _ in range(50):
        v = rng.integers(-3, 3, size=int(rng.integers(1, 40))).astype(np.float32)
        assert Sampler.greedy(v) == greedy_ref(v.tolist())


def test_migration_moves_the_requested_share_even_without_lower_holes():
    """Compaction stops at the first free id above the source; migration
    keeps going, so a fixed share of the live blocks moves (configs[4]'s
    relocation of 25% of the live blocks), with the data gathered unchanged."""
    rng = np.random.default_rng(5)
    nb, bs = 200, 16
    c = PagedCache(bs, nb)
    for sid in range(12):
        c.allocate(sid, int(rng.integers(50, 200)))
    live = sum(len(c.table(s)) for s in range(12))
    assert len(c.plan_compaction(1000)) == 0            # dense prefix: nothing to compact
    pool = rng.standard_normal((nb, 2, bs, 4)).astype(np.float32)
    before = {s: pool[c.table(s)].copy() for s in range(12)}
    want = live // 4
    pairs = c.plan_migration(want)
    assert len(pairs) == min(want, nb - live)
    src, dst = pairs[:, 0], pairs[:, 1]
    assert not set(src.tolist()) & set(dst.tolist())
    pool[dst] = pool[src]
    for s in range(12):
        np.testing.assert_array_equal(pool[c.table(s)], before[s])
    assert c.num_free() == nb - live


def test_relocation_fills_the_longest_free_runs_in_order():
    """plan_relocation moves what plan_migration moves (the highest live
    ids) into the longest runs of free ids, longest first, with both sides
    ascending; the data gathered through the tables is unchanged and the
    vacated sources join the free list."""
    rng = np.random.default_rng(7)
    nb, bs = 400, 16
    c, m = PagedCache(bs, nb), PagedCache(bs, nb)
    pending = {sid: int(rng.integers(3, 15)) for sid in range(20)}
    while pending:                                       # round-robin: interleaved ids
        for sid in list(pending):
            assert c.allocate(sid, bs) is not None and m.allocate(sid, bs) is not None
            pending[sid] -= 1
            if not pending[sid]:
                del pending[sid]
    for sid in (3, 8, 11):                               # single-block holes
        c.free(sid), m.free(sid)
    keep = [s for s in range(20) if s not in (3, 8, 11)]
    live = sum(len(c.table(s)) for s in keep)
    free_before = sorted(c.free_list())
    pool = rng.standard_normal((nb, 2, bs, 4)).astype(np.float32)
    before = {s: pool[c.table(s)].copy() for s in keep}
    want = live // 4
    pairs = c.plan_relocation(want)
    mig = m.plan_migration(want)
    assert len(pairs) == len(mig) == want
    src, dst = pairs[:, 0], pairs[:, 1]
    assert sorted(src.tolist()) == sorted(mig[:, 0].tolist())   # the same blocks move
    assert (np.diff(src) > 0).all() and (np.diff(dst) > 0).all()
    assert not set(src.tolist()) & set(dst.tolist())
    runs = []
    for f in free_before:
        if runs and runs[-1][0] + runs[-1][1] == f:
            runs[-1][1] += 1
        else:
            runs.append([f, 1])
    runs.sort(key=lambda r: (-r[1], r[0]))
    assert runs[0][1] >= want                            # the pool's unused top is one run
    assert dst.tolist() == list(range(runs[0][0], runs[0][0] + want))
    pool[dst] = pool[src]
    for s, v in before.items():
        np.testing.assert_array_equal(pool[c.table(s)], v)
    assert c.num_free() == nb - live
    free_after = set(c.free_list())
    assert set(src.tolist()) <= free_after and not set(dst.tolist()) & free_after
