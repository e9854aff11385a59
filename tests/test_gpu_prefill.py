"""GPU parity of causal prefill attention over the paged pool against the oracle.

Tolerances are those of decode attention: max-abs 1e-4 / rel 1e-3 against the
oracle on the same pool (fp32 and bf16 storage), and max-abs 2e-2 between a
bf16 pool and the oracle on the unrounded fp32 values.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from rustral_amd import kv
from tests.gpu_util import say, to_dev, to_np
from tests.helpers import assert_allclose_ref, make_pool, make_prefill, make_tables

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4
BF16_VS_F32_ATOL = 2e-2


def case(seed, hq, hkv, d, n_new, ctx, dtype, extra_blocks=3):
    rng = np.random.default_rng(seed)
    bs = 16
    nb = int(sum((int(c) + bs - 1) // bs for c in ctx)) + extra_blocks
    kp, vp, kf, vf = make_pool(rng, nb, hkv, bs, d, dtype)
    tables = make_tables(rng, ctx, bs, nb)
    qs = make_prefill(rng, n_new, ctx)
    q = rng.standard_normal((int(qs[-1]), hq, d)).astype(np.float32)
    return q, kp, vp, kf, vf, tables, qs


def run_gpu(dev, q, kp, vp, tables, qs, ctx, scale, max_q_len=None):
    out = kv.prefill_attention(to_dev(q, dev), to_dev(kp, dev), to_dev(vp, dev),
                               to_dev(tables, dev), to_dev(qs, dev), to_dev(ctx, dev), scale,
                               max_q_len=max_q_len)
    torch.cuda.synchronize()
    return to_np(out)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 2, 64), (4, 4, 32), (16, 2, 128),
                                      (8, 1, 64), (2, 1, 32)])
def test_prefill_shapes(dev, dtype, hq, hkv, d):
    """Square prefills (ctx == n), chunked prefills after cached tokens,
    single tokens, tiles that end mid-block, and a sequence without new tokens."""
    n_new = np.array([1, 16, 17, 40, 0, 128, 5, 33], np.int32)
    ctx = n_new + np.array([0, 0, 0, 100, 9, 0, 250, 47], np.int32)
    say(f"prefill dtype={dtype} hq={hq} hkv={hkv} d={d}")
    q, kp, vp, kf, vf, tables, qs = case(hq * 100 + d, hq, hkv, d, n_new, ctx, dtype)
    scale = float(np.float32(1.0 / math.sqrt(d)))
    got = run_gpu(dev, q, kp, vp, tables, qs, ctx, scale)
    want = oracle.prefill_attention(q, kp, vp, tables, qs, ctx, scale)
    assert_allclose_ref(got, want, RTOL, ATOL, "gpu vs oracle (same pool)")
    if dtype == "bf16":
        want32 = oracle.prefill_attention(q, kf, vf, tables, qs, ctx, scale)
        assert np.abs(got - want32).max() <= BF16_VS_F32_ATOL


def test_prefill_config4_admission_shape(dev):
    """configs[4]'s admissions: 25 sequences x 128 prompt tokens, Llama-3-8B
    layer shape (Hq 32, Hkv 8, D 128), bf16 pool."""
    n_new = np.full(25, 128, np.int32)
    say("prefill configs[4] admission shape 25 x 128")
    q, kp, vp, _, _, tables, qs = case(44, 32, 8, 128, n_new, n_new.copy(), "bf16")
    got = run_gpu(dev, q, kp, vp, tables, qs, n_new, 1 / math.sqrt(128))
    want = oracle.prefill_attention(q, kp, vp, tables, qs, n_new, 1 / math.sqrt(128))
    assert_allclose_ref(got, want, RTOL, ATOL, "gpu vs oracle")


def short_prefix_case(seed, n_seq, n_max, with_edges):
    """Ragged sequences of 1 .. n_max new tokens with at most as many cached
    keys as new ones (contexts up to 1.5 n_max); with_edges adds a sequence without new tokens and one
    with more new tokens than context (zero rows before position 0)."""
    rng = np.random.default_rng(seed)
    n_new = rng.integers(1, n_max + 1, size=n_seq).astype(np.int32)
    n_new[0] = n_max
    ctx = (n_new + rng.integers(0, n_new + 1)).astype(np.int32)
    ctx = np.minimum(ctx, n_max + n_max // 2).astype(np.int32)
    if with_edges:
        n_new[1], ctx[1] = 0, 30
        n_new[2], ctx[2] = 50, 20
    return n_new, ctx


# (seed, sequences, longest new-token run, edge sequences, Hq, Hkv, D, pool
# dtype, whether a wider table selects the 8-wave build).  bf16 pools: the
# 4-wave build on every call at D = 64 and at G = 1, on no call at G = 2 with
# D = 128, else for short cached prefixes; fp32 pools: every call at G = 1
# with D = 32, short cached prefixes at G = 1 with D = 128, else never.
SHORT_CASES = [(60, 40, 128, False, 32, 8, 128, "bf16", True),
               (61, 33, 96, True, 32, 8, 128, "bf16", True),
               (62, 7, 256, True, 32, 8, 128, "bf16", True),
               (63, 20, 128, True, 64, 8, 128, "bf16", True),
               (64, 30, 128, True, 32, 8, 64, "bf16", False),
               (65, 12, 160, True, 64, 8, 64, "bf16", False),
               (66, 40, 128, True, 32, 8, 32, "bf16", True),
               (67, 40, 128, True, 8, 8, 128, "bf16", False),
               (68, 40, 128, True, 16, 8, 64, "bf16", False),
               (69, 40, 128, True, 16, 8, 32, "bf16", True),
               (70, 25, 128, True, 16, 8, 128, "bf16", False),
               (71, 40, 128, True, 8, 8, 32, "f32", False),
               (72, 30, 128, True, 8, 8, 128, "f32", True),
               (73, 30, 128, True, 8, 8, 64, "bf16", False),
               (74, 30, 128, True, 8, 8, 64, "f32", False)]


@pytest.mark.parametrize("seed,n_seq,n_max,with_edges,hq,hkv,d,dtype,two_builds", SHORT_CASES)
def test_prefill_short_prefix_build(dev, seed, n_seq, n_max, with_edges, hq, hkv, d, dtype,
                                    two_builds):
    """The 4-wave build that touches the next round's q rows is taken on the
    calls it was measured faster for (per pool dtype, query heads per KV
    head and head_dim; for short cached prefixes the table width against the
    longest new-token run decides).  Grids of several hundred to a few
    thousand workgroups, over one to several rounds of the resident ones, so
    the touched rows include tiles past a sequence's end.  Against the
    oracle; where a wider table (extra -1 entries) selects the 8-wave build,
    bit-equal to it."""
    n_new, ctx = short_prefix_case(seed, n_seq, n_max, with_edges)
    say(f"prefill 4-wave build seed={seed} seqs={n_seq} n_max={n_max} hq={hq} d={d} {dtype}")
    q, kp, vp, _, _, tables, qs = case(seed, hq, hkv, d, n_new, ctx, dtype)
    assert tables.shape[1] * 16 <= 2 * int(n_new.max())
    scale = float(np.float32(1.0 / math.sqrt(d)))
    got = run_gpu(dev, q, kp, vp, tables, qs, ctx, scale)
    want = oracle.prefill_attention(q, kp, vp, tables, qs, ctx, scale)
    assert_allclose_ref(got, want, RTOL, ATOL, "gpu vs oracle")
    if with_edges:
        assert np.all(got[qs[2]:qs[2] + 30] == 0.0)
    wide = np.full((tables.shape[0], 2 * tables.shape[1] + 1), -1, np.int32)
    wide[:, :tables.shape[1]] = tables
    other = run_gpu(dev, q, kp, vp, wide, qs, ctx, scale)
    if two_builds:
        assert np.array_equal(got, other)
    else:
        assert_allclose_ref(other, want, RTOL, ATOL, "gpu (wide table) vs oracle")
    # the rows past a max_q_len cap stay unwritten in the 4-wave build too
    # (the cap still at least half the table's keys)
    cap = (tables.shape[1] * 16 + 1) // 2
    assert cap < n_max
    capped = run_gpu(dev, q, kp, vp, tables, qs, ctx, scale, max_q_len=cap)
    rows = np.concatenate([np.arange(qs[b], qs[b] + min(cap, n_new[b])) for b in range(n_seq)])
    assert np.array_equal(capped[rows], got[rows])
    assert np.all(capped[np.setdiff1d(np.arange(qs[-1]), rows)] == 0.0)


def test_prefill_long_chunk_after_long_context(dev):
    n_new = np.array([200, 64], np.int32)
    ctx = np.array([3000, 1100], np.int32)
    say("prefill chunk of 200 after 2800 cached tokens")
    q, kp, vp, _, _, tables, qs = case(45, 8, 2, 128, n_new, ctx, "bf16")
    got = run_gpu(dev, q, kp, vp, tables, qs, ctx, 0.09)
    want = oracle.prefill_attention(q, kp, vp, tables, qs, ctx, 0.09)
    assert_allclose_ref(got, want, RTOL, ATOL, "gpu vs oracle")


def test_prefill_last_token_equals_gpu_decode(dev):
    """The last new token of each sequence attends to its whole context: the
    prefill row equals the decode kernel's output for that query."""
    n_new = np.array([37, 16, 1, 90], np.int32)
    ctx = np.array([37, 500, 70, 1200], np.int32)
    say("prefill last token vs decode")
    q, kp, vp, _, _, tables, qs = case(46, 32, 8, 128, n_new, ctx, "bf16")
    got = run_gpu(dev, q, kp, vp, tables, qs, ctx, 0.088)
    last = qs[1:] - 1
    dec = kv.decode_attention(to_dev(np.ascontiguousarray(q[last]), dev), to_dev(kp, dev),
                              to_dev(vp, dev), to_dev(tables, dev), to_dev(ctx, dev), 0.088)
    torch.cuda.synchronize()
    assert_allclose_ref(got[last], to_np(dec), RTOL, ATOL, "prefill last row vs decode")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_prefill_invalid_blocks_and_short_context(dev, dtype):
    """Blocks with an out-of-range id are left out; more new tokens than
    context gives zero rows before position 0; rows past max_q_len are not
    written."""
    n_new = np.array([40, 6, 20], np.int32)
    ctx = np.array([300, 4, 20], np.int32)
    say(f"prefill invalid blocks / short context dtype={dtype}")
    q, kp, vp, _, _, tables, qs = case(47, 8, 2, 64, n_new, ctx, dtype)
    nb = kp.shape[0]
    tables = tables.copy()
    tables[0, 3] = nb + 7
    tables[0, 10] = -5
    got = run_gpu(dev, q, kp, vp, tables, qs, ctx, 0.125)
    want = oracle.prefill_attention(q, kp, vp, tables, qs, ctx, 0.125)
    assert_allclose_ref(got, want, RTOL, ATOL, "gpu vs oracle")
    assert np.all(got[qs[1]:qs[1] + 2] == 0.0)
    capped = run_gpu(dev, q, kp, vp, tables, qs, ctx, 0.125, max_q_len=16)
    rows = np.concatenate([np.arange(qs[b], qs[b] + min(16, n_new[b])) for b in range(3)])
    assert np.array_equal(capped[rows], got[rows])
    unwritten = np.setdiff1d(np.arange(qs[-1]), rows)
    assert np.all(capped[unwritten] == 0.0)


def test_prefill_no_new_tokens_is_a_no_op(dev):
    say("prefill with no new tokens")
    q, kp, vp, _, _, tables, qs = case(48, 4, 2, 32, np.array([0, 0], np.int32),
                                       np.array([10, 20], np.int32), "bf16")
    q = np.zeros((4, 4, 32), np.float32)
    got = run_gpu(dev, q, kp, vp, tables, qs, np.array([10, 20], np.int32), 0.1, max_q_len=0)
    assert np.all(got == 0.0)
