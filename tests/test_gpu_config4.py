"""configs[4], the continuous-batching step mix, on the GPU at its shape with
2 layers: 256 running sequences with contexts U[1, 8192] in a pool of 84,000
16-token blocks per layer (bf16, Hkv 8, D 128, Hq 32), blocks handed out
round-robin so sequences interleave.  One step:

1. 10% of the sequences finish (blocks freed);
2. the block manager plans the relocation of 25% of the live blocks
   (rkv_bm_plan_relocation, into the longest free runs, as bench.py's
   configs[4] step does) and copy_blocks moves them in both layers; then a
   further 10% by rkv_bm_plan_migration (into the lowest free ids); every
   live sequence's gather is bit-equal before and after each;
3. 10% new sequences are admitted with 128-token prefills appended in bulk
   and run through causal prefill attention: within 1e-4 / 1e-3 of the
   oracle on the same bf16 pool;
4. one decode token per running sequence: appended, then decode attention
   over every sequence, every one checked against the oracle.

The caller this replaces is ServingEngine::step, which runs no model forward
(crates/nn/src/continuous_batching.rs:516-528).
"""
import math

import numpy as np
import pytest
import torch

import oracle
from rustral_amd import kv
from rustral_amd.serving import PagedCache
from tests.gpu_util import say, to_np
from tests.helpers import assert_allclose_ref

pytestmark = pytest.mark.gpu

L_, NB, B, PRE, HKV, HQ, D, BS = 2, 84000, 256, 128, 8, 32, 128, 16


def _mini_pool(kp, vp, tables_rows):
    """The blocks of the given table rows copied to the host by torch indexing
    (independent of the library's gather), with tables renumbered 0..n-1."""
    ids = sorted({int(b) for row in tables_rows for b in row if b >= 0})
    remap = {b: i for i, b in enumerate(ids)}
    idx = torch.tensor(ids, dtype=torch.int64, device=kp.device)
    k = to_np(kp.index_select(0, idx).contiguous())
    v = to_np(vp.index_select(0, idx).contiguous())
    mb = max(len(r) for r in tables_rows)
    t = np.full((len(tables_rows), mb), -1, np.int32)
    for i, row in enumerate(tables_rows):
        t[i, :len(row)] = [remap[int(b)] for b in row]
    return k, v, t


def test_config4_step_mix(dev):
    say("configs[4] step mix, 2 layers, 84,000-block pools")
    rng = np.random.default_rng(4)
    g = torch.Generator(device=dev).manual_seed(4)
    kp = torch.randn((L_, NB, HKV, BS, D), generator=g, device=dev).to(torch.bfloat16)
    vp = torch.randn((L_, NB, HKV, BS, D), generator=g, device=dev).to(torch.bfloat16)
    cache = PagedCache(BS, NB)
    ctx = {i: int(c) for i, c in enumerate(rng.integers(1, 8192 + 1, size=B))}
    pending = {i: -(-c // BS) for i, c in ctx.items()}
    while pending:                                   # round-robin: sequences interleave
        for i in list(pending):
            assert cache.allocate(i, BS) is not None
            pending[i] -= 1
            if pending[i] == 0:
                del pending[i]
    n_turn = B // 10
    scale = 1.0 / math.sqrt(D)

    # 1. finish 10%
    for i in rng.choice(sorted(ctx), size=n_turn, replace=False).tolist():
        cache.free(i)
        del ctx[i]
    ids = sorted(ctx)
    live = sum(len(cache.table(i)) for i in ids)

    def gather_all():
        mb = max(len(cache.table(i)) for i in ids)
        t = torch.from_numpy(cache.fill_tables(ids, mb)).to(dev)
        c = torch.tensor([ctx[i] for i in ids], dtype=torch.int32, device=dev)
        offs = np.concatenate([[0], np.cumsum([ctx[i] * HKV * D for i in ids])[:-1]]).astype(np.int64)
        total = int(sum(ctx[i] for i in ids)) * HKV * D
        out = []
        for layer in range(L_):
            out.append(kv.gather(kp[layer], vp[layer], t, c, out_offsets=torch.from_numpy(offs).to(dev),
                                 out_total=total))
        return out

    before = gather_all()
    # 2. relocate 25% of the live blocks (both layers, K and V), then 10% more
    for plan, share in ((cache.plan_relocation, 4), (cache.plan_migration, 10)):
        pairs = plan(live // share)
        say(f"{plan.__name__}: {len(pairs)} of {live} live blocks")
        assert len(pairs) == live // share
        assert not set(pairs[:, 0].tolist()) & set(pairs[:, 1].tolist())
        kv.copy_blocks(kp, vp, torch.from_numpy(pairs).to(dev))
        after = gather_all()
        torch.cuda.synchronize()
        for layer in range(L_):
            for a, b in zip(before[layer], after[layer]):
                assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"layer {layer}"
        del after
    del before

    # 3. admit 10% with 128-token prefills, appended in bulk, causal prefill
    admitted = list(range(10_000, 10_000 + n_turn))
    for i in admitted:
        assert cache.allocate(i, PRE) is not None
        ctx[i] = PRE
    slots = np.concatenate([np.asarray(cache.table(i), np.int64)[np.arange(PRE) // BS] * BS
                            + np.arange(PRE) % BS for i in admitted])
    kn = torch.randn((L_, n_turn * PRE, HKV, D), generator=g, device=dev)
    vn = torch.randn_like(kn)
    kv.append(kp, vp, kn, vn, torch.from_numpy(slots).to(dev))
    q_pre = torch.randn((n_turn * PRE, HQ, D), generator=g, device=dev)
    tab_pre = cache.fill_tables(admitted, PRE // BS)
    qs = torch.arange(0, (n_turn + 1) * PRE, PRE, dtype=torch.int32, device=dev)
    cpre = torch.full((n_turn,), PRE, dtype=torch.int32, device=dev)
    for layer in range(L_):
        out = kv.prefill_attention(q_pre, kp[layer], vp[layer], torch.from_numpy(tab_pre).to(dev), qs,
                                   cpre, scale, max_q_len=PRE)
        k_h, v_h, t_h = _mini_pool(kp[layer], vp[layer], [cache.table(i) for i in admitted])
        want = oracle.prefill_attention(to_np(q_pre), k_h, v_h, t_h,
                                        np.arange(0, (n_turn + 1) * PRE, PRE, dtype=np.int32),
                                        np.full(n_turn, PRE, np.int32), scale)
        assert_allclose_ref(to_np(out), want, 1e-3, 1e-4, f"prefill layer {layer}")

    # 4. one decode token per running sequence
    ids = sorted(ctx)
    for i in ids:
        assert cache.reserve(i, ctx[i] + 1) >= 0
    mb = max(len(cache.table(i)) for i in ids)
    tables = cache.fill_tables(ids, mb)
    pos = np.array([ctx[i] for i in ids], np.int64)
    slots_dec = tables[np.arange(len(ids)), pos // BS].astype(np.int64) * BS + pos % BS
    kd = torch.randn((L_, len(ids), HKV, D), generator=g, device=dev)
    vd = torch.randn_like(kd)
    kv.append(kp, vp, kd, vd, torch.from_numpy(slots_dec).to(dev))
    cl = (pos + 1).astype(np.int32)
    q = torch.randn((len(ids), HQ, D), generator=g, device=dev)
    check = np.arange(len(ids))
    for layer in range(L_):
        out = kv.decode_attention(q, kp[layer], vp[layer], torch.from_numpy(tables).to(dev),
                                  torch.from_numpy(cl).to(dev), scale, max_context=mb * BS)
        k_h, v_h, t_h = _mini_pool(kp[layer], vp[layer], [cache.table(ids[j]) for j in check])
        want = oracle.decode_attention(to_np(q)[check], k_h, v_h, t_h, cl[check], scale, n_threads=16)
        assert_allclose_ref(to_np(out)[check], want, 1e-3, 1e-4, f"decode layer {layer}")
