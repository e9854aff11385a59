"""The device-side block manager (rkv_dbm_*) against the oracle's restatement
of PagedCache (oracle/serving_ref.PagedCacheRef, kv_cache.rs:381-432) and
the product's host manager (rkv_bm_*): the same calls give the same block
ids in the same tables and the same free-list order (bit-exact) in all
three, failures change nothing,
and a decode step driven entirely from device memory -- reserve, slot
mapping, append, batch tables, attention -- equals the same step driven by
host-built tables.  A HIP-graph replay of reserve + slot mapping matches the
eager host results at every replay.
"""
import math

import numpy as np
import pytest
import torch

from oracle.serving_ref import PagedCacheRef
from rustral_amd import kv
from rustral_amd.serving import PagedCache
from tests.gpu_util import say

pytestmark = pytest.mark.gpu

ERR_OOM, ERR_TABLE_FULL, ERR_ARG = 1, 2, 4


class Managers:
    """The oracle's PagedCacheRef and the product host manager, driven by
    the same calls; reserve reports None on OOM in both."""

    def __init__(self, bs, nb):
        self.ref, self.host = PagedCacheRef(bs, nb), PagedCache(bs, nb)

    def reserve(self, seq, tokens):
        a, b = self.ref.reserve(seq, tokens), self.host.reserve(seq, tokens)
        assert (a is None) == (b is None), (seq, tokens, a, b)
        return a

    def free(self, seq):
        assert self.ref.free(seq) == self.host.free(seq)

    def table(self, seq):
        return self.ref.table(seq)

    def num_free(self):
        return len(self.ref.free_blocks)

    def fill_tables(self, seqs, width):
        t = np.full((len(seqs), width), -1, np.int32)
        for i, s in enumerate(seqs):
            row = self.ref.table(s)
            t[i, :len(row)] = row
        return t


def assert_same_state(dbm, mgr, slots_in_use):
    tables, lengths, free = dbm.download()
    assert free.tolist() == mgr.ref.free_blocks, "free list order vs the oracle"
    assert mgr.host.free_list() == mgr.ref.free_blocks, "free list order: host vs the oracle"
    for s in range(dbm.max_seqs):
        want = mgr.ref.table(s) if s in slots_in_use else []
        assert mgr.host.table(s) == want, f"slot {s}: host table vs the oracle"
        assert lengths[s] == len(want), f"slot {s} length"
        assert tables[s, :len(want)].tolist() == want, f"slot {s} table"
        assert (tables[s, len(want):] == -1).all(), f"slot {s} tail"


def test_random_trace_matches_host_manager(dev):
    say("device block manager: random trace vs host")
    rng = np.random.default_rng(5)
    nb, bs, max_seqs, max_blocks = 400, 16, 40, 64
    dbm = kv.DeviceBlockManager(nb, bs, max_seqs, max_blocks, device=dev)
    host = Managers(bs, nb)
    lens = {}
    for step in range(60):
        if lens and rng.random() < 0.25:
            gone = rng.choice(sorted(lens), size=rng.integers(1, len(lens) + 1), replace=False)
            gone = [int(x) for x in gone]
            dbm.free(gone)
            for s in gone:
                host.free(s)
                del lens[s]
        else:
            k = int(rng.integers(1, 12))
            slots = [int(x) for x in rng.choice(max_seqs, size=k, replace=False)]
            toks = []
            for s in slots:
                lens[s] = lens.get(s, 0) + int(rng.integers(0, 70))
                toks.append(lens[s])
            need = sum(max(0, -(-t // bs) - len(host.table(s))) for s, t in zip(slots, toks))
            if need > host.num_free():  # keep the trace inside the pool
                for s, t in zip(slots, toks):
                    lens[s] = len(host.table(s)) * bs if host.table(s) else 0
                    if lens[s] == 0:
                        del lens[s]
                continue
            dbm.reserve(slots, toks)
            for s, t in zip(slots, toks):
                assert host.reserve(s, t) is not None
        nf, err = dbm.status()
        assert err == 0 and nf == host.num_free()
        assert_same_state(dbm, host, set(lens))
    dbm.close()


def test_reserve_is_all_or_nothing(dev):
    say("device block manager: OOM / table full / bad slot change nothing")
    nb, bs = 20, 16
    dbm = kv.DeviceBlockManager(nb, bs, 8, 16, device=dev)
    host = Managers(bs, nb)
    dbm.reserve([0, 1], [100, 150])              # 7 + 10 blocks
    host.reserve(0, 100), host.reserve(1, 150)
    before = dbm.download()
    dbm.reserve([2, 3], [16, 64])                 # needs 1 + 4 > 3 free: OOM
    nf, err = dbm.status()
    assert err & ERR_OOM and nf == 3
    after = dbm.download()
    assert all(np.array_equal(a, b) for a, b in zip(before, after))
    assert dbm.status(clear=True)[1] != 0 and dbm.status()[1] == 0
    dbm.reserve([4], [17 * bs])                   # 17 blocks > max_blocks 16
    assert dbm.status(clear=True)[1] & ERR_TABLE_FULL
    dbm.reserve([9], [16])                        # slot outside [0, 8)
    assert dbm.status(clear=True)[1] & ERR_ARG
    dbm.free([-1])
    assert dbm.status(clear=True)[1] & ERR_ARG
    assert_same_state(dbm, host, {0, 1})
    dbm.reserve([2, 3], [16, 32])                 # 1 + 2 = 3 free: fits exactly
    host.reserve(2, 16), host.reserve(3, 32)
    assert dbm.status() == (0, 0)
    assert_same_state(dbm, host, {0, 1, 2, 3})
    dbm.close()


def test_repeated_slot_fails_the_call(dev):
    """A slot twice in one reserve or free -- within one 1024-thread chunk of
    the call or in different chunks -- fails the call with ERR_ARG and
    changes nothing; later calls behave as the host's (the repeat check
    leaves no marks in the lengths)."""
    say("device block manager: repeated slots fail the call")
    nb, bs, max_seqs = 3000, 16, 1500
    dbm = kv.DeviceBlockManager(nb, bs, max_seqs, 8, device=dev)
    host = Managers(bs, nb)
    dbm.reserve([0, 1], [20, 40])
    host.reserve(0, 20), host.reserve(1, 40)
    before = dbm.download()
    for slots in ([2, 5, 2], [1, 0], list(range(2, 1300)) + [7]):
        dbm.reserve(slots, [16] * len(slots))
        if slots == [1, 0]:                       # distinct, no growth: a no-op
            assert dbm.status() == (host.num_free(), 0)
        else:
            assert dbm.status(clear=True)[1] == ERR_ARG
        assert all(np.array_equal(x, y) for x, y in zip(before, dbm.download()))
    dbm.free([1, 0, 1])
    assert dbm.status(clear=True)[1] == ERR_ARG
    assert all(np.array_equal(x, y) for x, y in zip(before, dbm.download()))
    slots = list(range(2, 1300))
    dbm.reserve(slots, [16] * len(slots))
    for s in slots:
        host.reserve(s, 16)
    assert dbm.status() == (host.num_free(), 0)
    assert_same_state(dbm, host, {0, 1, *slots})
    dbm.free([1, 0])
    host.free(1), host.free(0)
    assert dbm.status() == (host.num_free(), 0)
    assert_same_state(dbm, host, set(slots))
    dbm.close()


def test_device_resident_decode_step_equals_host_driven_step(dev):
    """Prompts of 1..300 tokens, then 3 decode steps; all of it from device
    memory vs the same steps with host-built slots and tables."""
    say("device-resident decode step vs host-driven step")
    rng = np.random.default_rng(8)
    nb, bs, hkv, hq, d, B = 200, 16, 2, 8, 64, 6
    max_blocks = 32
    prompt = rng.integers(1, 300, B).astype(np.int32)
    scale = 1.0 / math.sqrt(d)
    pools = [torch.zeros((nb, hkv, bs, d), dtype=torch.bfloat16, device=dev) for _ in range(4)]
    dbm = kv.DeviceBlockManager(nb, bs, 16, max_blocks, device=dev)
    host = Managers(bs, nb)
    slots = list(range(3, 3 + B))
    lens = prompt.copy()
    outs = []
    for step in range(4):
        n_new = lens if step == 0 else np.ones(B, np.int32)
        start = np.zeros(B, np.int32) if step == 0 else lens - 1
        tot = int(n_new.sum())
        k_new = torch.randn((tot, hkv, d), device=dev)
        v_new = torch.randn((tot, hkv, d), device=dev)
        seq_of = np.repeat(np.arange(B), n_new)
        pos = np.concatenate([np.arange(s, s + n) for s, n in zip(start, n_new)]).astype(np.int32)
        # device-driven
        dbm.reserve(slots, lens)
        dslots = dbm.slot_mapping([slots[b] for b in seq_of], pos)
        kv.append(pools[0], pools[1], k_new, v_new, dslots)
        dtab = dbm.batch_tables(slots, max_blocks)
        # host-driven
        hslots = []
        for b in range(B):
            host.reserve(slots[b], int(lens[b]))
        for b, p in zip(seq_of, pos):
            t = host.table(slots[b])
            hslots.append(t[p // bs] * bs + p % bs)
        assert torch.equal(dslots.cpu(), torch.tensor(hslots, dtype=torch.int64))
        kv.append(pools[2], pools[3], k_new, v_new,
                  torch.tensor(hslots, dtype=torch.int64, device=dev))
        htab = torch.as_tensor(host.fill_tables(slots, max_blocks), device=dev)
        assert torch.equal(dtab, htab)
        q = torch.randn((B, hq, d), device=dev)
        ctx = torch.as_tensor(lens, dtype=torch.int32, device=dev)
        o_dev = kv.decode_attention(q, pools[0], pools[1], dtab, ctx, scale,
                                    max_context=max_blocks * bs)
        o_host = kv.decode_attention(q, pools[2], pools[3], htab, ctx, scale,
                                     max_context=max_blocks * bs)
        torch.cuda.synchronize()
        assert torch.equal(pools[0], pools[2]) and torch.equal(pools[1], pools[3])
        assert torch.equal(o_dev, o_host)
        outs.append(o_dev)
        lens = lens + 1
    assert dbm.status() == (host.num_free(), 0)
    dbm.close()


def test_graph_replay_of_reserve_and_slot_mapping(dev):
    """reserve + slot mapping captured once, replayed for 6 steps with the
    token counts updated in place between replays (eager work and a
    synchronisation between replays); tables and slots equal the host's."""
    say("device block manager under HIP graph replay")
    nb, bs, B, max_blocks = 120, 16, 5, 24
    dbm = kv.DeviceBlockManager(nb, bs, 8, max_blocks, device=dev)
    host = Managers(bs, nb)
    slots = torch.tensor([1, 4, 2, 7, 0], dtype=torch.int32, device=dev)
    lens = np.array([15, 16, 17, 40, 1], np.int32)
    ntok = torch.tensor(lens, dtype=torch.int32, device=dev)
    pos = torch.tensor(lens - 1, dtype=torch.int32, device=dev)
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            dbm.reserve(slots, ntok)
            out = dbm.slot_mapping(slots, pos)
    torch.cuda.synchronize(dev)
    for step in range(6):
        ntok.copy_(torch.tensor(lens, dtype=torch.int32))
        pos.copy_(torch.tensor(lens - 1, dtype=torch.int32))
        torch.cuda.synchronize(dev)
        g.replay()
        torch.cuda.synchronize(dev)
        want = []
        for s, n in zip(slots.tolist(), lens.tolist()):
            host.reserve(s, n)
            t = host.table(s)
            want.append(t[(n - 1) // bs] * bs + (n - 1) % bs)
        assert out.cpu().tolist() == want, f"replay {step}"
        assert dbm.status()[1] == 0
        assert_same_state(dbm, host, set(slots.tolist()))
        lens = lens + np.array([1, 7, 16, 3, 30], np.int32)
    dbm.close()
