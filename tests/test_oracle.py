"""Pins the CPU oracle (oracle/rkv_oracle.c) before anything is compared with it.

Each check is chosen to fail on a plausible slip (dropped term, wrong index,
transposed operand, wrong rounding): reference known answers
(tests/golden/reference_kats.json), an independent float64 numpy
formulation, torch library routines, closed forms and invariants.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_allclose_ref, contexts, make_pool, make_tables, ref_decode_f64

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
KATS = json.load(open(os.path.join(GOLDEN, "reference_kats.json")))


# ---- bf16 conversion ---------------------------------------------------------

def test_bf16_rne_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
        # exact ties: low 16 bits 0x8000 with even/odd bit 16
        np.array([0x3f808000, 0x3f818000, 0xbf808000, 0x00008000, 0x7f7f8000, 0x7f7fffff,
                  0x00000001, 0x807fffff], dtype=np.uint32).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 1.01171875], np.float32),
    ])
    got = oracle.bf16_from_f32(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    assert oracle.bf16_from_f32(np.float32([1.01171875]))[0] == 0x3F82  # -> 1.015625


def test_bf16_nan_stays_nan_and_upcast_is_exact():
    nan = np.array([0x7fc00000, 0xffc00001, 0x7f800001], np.uint32).view(np.float32)
    b = oracle.bf16_from_f32(nan)
    assert np.isnan(oracle.f32_from_bf16(b)).all()
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    up = oracle.f32_from_bf16(bits)
    fin = np.isfinite(up)
    assert np.array_equal(oracle.bf16_from_f32(up[fin]), bits[fin])  # round trip is the identity
    assert np.array_equal(up.view(np.uint32), bits.astype(np.uint32) << 16)


# ---- softmax / argmax (reference known answers) ------------------------------

def test_softmax_rows_reference_golden():
    k = KATS["softmax_dim1"]
    x = np.array(k["input"], np.float32).reshape(k["rows"], k["cols"])
    got = oracle.softmax_rows(x)
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    want = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    assert_allclose_ref(got, want, k["tolerance"]["rtol"], k["tolerance"]["atol"], "softmax")
    assert np.allclose(got.sum(axis=1), 1.0, atol=1e-6)


def _softmax_f64(x, axis):
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=axis, keepdims=True))
    return e / e.sum(axis=axis, keepdims=True)


def test_softmax_dim_reference_golden_and_every_axis():
    k = KATS["softmax_dim1"]
    x = np.array(k["input"], np.float32).reshape(k["rows"], k["cols"])
    tol = (k["tolerance"]["rtol"], k["tolerance"]["atol"])
    assert_allclose_ref(oracle.softmax_dim(x, 1), _softmax_f64(x, 1).astype(np.float32), *tol,
                        "softmax_dim golden")
    # a 3-d tensor of distinct sizes: each axis against numpy's along that axis,
    # so an outer/inner stride slip or a wrong axis fails
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((3, 5, 7)) * 4).astype(np.float32)
    for dim in range(3):
        got = oracle.softmax_dim(x, dim)
        assert_allclose_ref(got, _softmax_f64(x, dim).astype(np.float32), *tol, f"dim {dim}")
        assert np.allclose(got.sum(axis=dim), 1.0, atol=1e-6)
    with pytest.raises(ValueError):
        oracle.softmax_dim(np.zeros((2, 0), np.float32), 1)  # axis size 0 (lib.rs:1200-1202)


def test_softmax_dim_nan_and_infinity_rules():
    # f32::max skips a NaN operand, so the max is that of the other entries;
    # exp(NaN - max) then makes the sum, and the whole line, NaN
    y = oracle.softmax_dim(np.float32([[1.0, np.nan, 2.0]]), 1)
    assert np.isnan(y).all()
    # an all -inf line: max -inf, exp(-inf - -inf) = NaN
    assert np.isnan(oracle.softmax_dim(np.full((1, 4), -np.inf, np.float32), 1)).all()
    # a -inf entry among finite ones gets weight exactly 0
    y = oracle.softmax_dim(np.float32([[0.0, -np.inf, 3.0]]), 1)
    assert y[0, 1] == 0.0 and np.isclose(y[0].sum(), 1.0)


def test_matmul_transpose_mul_scalar():
    k = KATS["matmul_2x2"]
    a = np.array(k["a"], np.float32).reshape(k["shape"])
    b = np.array(k["b"], np.float32).reshape(k["shape"])
    assert oracle.matmul(a, b).ravel().tolist() == k["expected"]
    rng = np.random.default_rng(6)
    a = rng.standard_normal((9, 37)).astype(np.float32)
    b = rng.standard_normal((37, 13)).astype(np.float32)
    y = oracle.matmul(a, b)
    want = a.astype(np.float64) @ b.astype(np.float64)
    assert np.abs(y - want).max() < 1e-4 * np.abs(want).max()
    # the serial order: row i of y is the float32 left-to-right sum of its products
    for i, j in [(0, 0), (8, 12), (4, 7)]:
        s = np.float32(0)
        for kk in range(37):
            s = np.float32(s + np.float32(a[i, kk] * b[kk, j]))
        assert y[i, j] == s
    assert np.array_equal(oracle.matmul(a, np.eye(37, dtype=np.float32)), a)  # identity
    assert np.array_equal(oracle.transpose(a), a.T)
    assert np.array_equal(oracle.mul_scalar(a, 0.125), a * np.float32(0.125))


def test_argmax_reference_and_ties():
    g = KATS["greedy"]
    assert oracle.argmax(g["logits"]) == g["expected"]
    assert oracle.argmax([1.0, 3.0, 3.0, 0.0]) == 2  # max_by keeps the last maximum
    assert oracle.argmax([5.0] * 7) == 6
    assert oracle.argmax([2.0]) == 0
    assert oracle.argmax([]) == -1


# ---- append / gather / copy: independent numpy indexing ----------------------

@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_append_matches_fancy_indexing(dtype):
    rng = np.random.default_rng(1)
    nb, hkv, bs, d = 20, 3, 16, 32
    canary = 7.0
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d, dtype, canary=canary)
    n = 50
    slots = rng.permutation(nb * bs)[:n].astype(np.int64)
    slots[3] = -1            # padding token
    slots[9] = nb * bs + 5   # out of range
    kn = rng.standard_normal((n, hkv, d)).astype(np.float32)
    vn = rng.standard_normal((n, hkv, d)).astype(np.float32)
    oracle.append(kp, vp, kn, vn, slots)
    keep = (slots >= 0) & (slots < nb * bs)
    blk, row = slots[keep] // bs, slots[keep] % bs
    conv = (lambda a: a) if dtype == "f32" else (
        lambda a: torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(kp[blk, :, row, :], conv(kn[keep]))
    assert np.array_equal(vp[blk, :, row, :], conv(vn[keep]))
    mask = np.ones((nb, bs), bool)
    mask[blk, row] = False
    can = np.float32(canary) if dtype == "f32" else oracle.bf16_from_f32(np.float32([canary]))[0]
    assert (kp.transpose(0, 2, 1, 3)[mask] == can).all()


def test_append_head_major_source_strides():
    """new_k in the KVCache layout [1, Hkv, T, D] (kv_cache.rs:173) via strides."""
    rng = np.random.default_rng(2)
    nb, hkv, bs, d, T = 8, 2, 16, 32, 20
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d, canary=0.0)
    kn = rng.standard_normal((hkv, T, d)).astype(np.float32)
    slots = np.arange(T, dtype=np.int64) + 16 * 3
    oracle.append(kp, vp, kn, kn, slots, tok_stride=d, head_stride=T * d)
    for t in range(T):
        assert np.array_equal(kp[3 + t // 16, :, t % 16, :], kn[:, t, :])


@pytest.mark.parametrize("out_f32", [False, True])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_gather_matches_fancy_indexing_and_roundtrip(dtype, out_f32):
    rng = np.random.default_rng(3)
    nb, hkv, bs, d = 64, 2, 16, 64
    ctx = np.array([0, 1, 16, 17, 100], np.int32)
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d, dtype)
    tables = make_tables(rng, ctx, bs, nb)
    ko, vo = oracle.gather(kp, vp, tables, ctx, out_f32=out_f32)
    for b, L in enumerate(ctx):
        pos = np.arange(L)
        want = kp[tables[b, pos // bs], :, pos % bs, :].transpose(1, 0, 2)
        if out_f32:
            want = oracle.pool_as_f32(want)
        assert np.array_equal(ko[b, :, :L], want)
        assert not ko[b, :, L:].any()  # rows past L untouched (zeros)
    # packed layout: offsets = prefix sums of Hkv*L*D
    sizes = ctx.astype(np.int64) * hkv * d
    off = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    kk, vv = oracle.gather(kp, vp, tables, ctx, out_offsets=off, out_f32=out_f32)
    for b, L in enumerate(ctx):
        assert np.array_equal(kk[off[b]:off[b] + sizes[b]].reshape(hkv, L, d), ko[b, :, :L])
        assert np.array_equal(vv[off[b]:off[b] + sizes[b]].reshape(hkv, L, d), vo[b, :, :L])


def test_gather_of_append_is_identity():
    rng = np.random.default_rng(4)
    nb, hkv, bs, d = 40, 4, 16, 32
    ctx = np.array([5, 33, 48], np.int32)
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d, canary=0.0)
    tables = make_tables(rng, ctx, bs, nb)
    xs = []
    for b, L in enumerate(ctx):
        pos = np.arange(L)
        slots = tables[b, pos // bs].astype(np.int64) * bs + pos % bs
        x = rng.standard_normal((L, hkv, d)).astype(np.float32)
        oracle.append(kp, vp, x, -x, slots)
        xs.append(x)
    ko, vo = oracle.gather(kp, vp, tables, ctx)
    for b, L in enumerate(ctx):
        assert np.array_equal(ko[b, :, :L], xs[b].transpose(1, 0, 2))
        assert np.array_equal(vo[b, :, :L], -xs[b].transpose(1, 0, 2))


def test_copy_blocks_multi_layer():
    rng = np.random.default_rng(5)
    nl, nb, hkv, bs, d = 3, 30, 2, 16, 32
    kp = rng.standard_normal((nl, nb, hkv, bs, d)).astype(np.float32)
    vp = rng.standard_normal((nl, nb, hkv, bs, d)).astype(np.float32)
    k0, v0 = kp.copy(), vp.copy()
    perm = rng.permutation(nb)
    pairs = np.stack([perm[:8], perm[8:16]], axis=1).astype(np.int32)
    pairs = np.concatenate([pairs, [[0, nb + 3], [-1, 2]]]).astype(np.int32)  # skipped entries
    oracle.copy_blocks(kp, vp, pairs)
    want_k, want_v = k0.copy(), v0.copy()
    want_k[:, perm[8:16]] = k0[:, perm[:8]]
    want_v[:, perm[8:16]] = v0[:, perm[:8]]
    assert np.array_equal(kp, want_k) and np.array_equal(vp, want_v)


# ---- decode attention ---------------------------------------------------------

def test_decode_matches_committed_golden():
    g = np.load(os.path.join(GOLDEN, "decode_small.npz"))
    got = oracle.decode_attention(g["q"], g["k_pool"], g["v_pool"], g["tables"], g["ctx_lens"],
                                  float(g["scale"]))
    assert_allclose_ref(got, g["expected"], 1e-5, 1e-6, "golden")
    got64 = oracle.decode_attention(g["q"], g["k_pool"], g["v_pool"], g["tables"], g["ctx_lens"],
                                    float(g["scale"]), f64=True)
    assert np.abs(got64 - g["expected"]).max() < 1e-12


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("hq,hkv,d", [(4, 4, 32), (8, 2, 64), (32, 8, 128), (8, 1, 128)])
def test_decode_vs_independent_f64(dtype, hq, hkv, d):
    rng = np.random.default_rng(hq * 100 + d)
    bs = 16
    ctx = np.array([1, 2, 15, 16, 17, 100, 257], np.int32)
    nb = int(sum((c + bs - 1) // bs for c in ctx)) + 3
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d, dtype)
    tables = make_tables(rng, ctx, bs, nb)
    q = rng.standard_normal((len(ctx), hq, d)).astype(np.float32)
    scale = float(np.float32(1.0 / math.sqrt(d)))  # the ABI takes a float32 scale
    got = oracle.decode_attention(q, kp, vp, tables, ctx, scale)
    want = ref_decode_f64(q, oracle.pool_as_f32(kp), oracle.pool_as_f32(vp), tables, ctx, scale)
    assert_allclose_ref(got, want, 1e-4, 1e-5, "f32 oracle vs numpy f64")
    got64 = oracle.decode_attention(q, kp, vp, tables, ctx, scale, f64=True)
    assert np.abs(got64 - want).max() < 1e-10


def test_decode_vs_torch_sdpa():
    """torch's scaled_dot_product_attention (float64, CPU) on the gathered K/V."""
    rng = np.random.default_rng(6)
    B, hq, hkv, d, bs = 4, 8, 2, 64, 16
    ctx = np.array([3, 40, 64, 129], np.int32)
    nb = 30
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d)
    tables = make_tables(rng, ctx, bs, nb)
    q = rng.standard_normal((B, hq, d)).astype(np.float32)
    got = oracle.decode_attention(q, kp, vp, tables, ctx, 0.125)
    ko, vo = oracle.gather(kp, vp, tables, ctx)
    for b, L in enumerate(ctx):
        K = torch.from_numpy(ko[b, :, :L]).double().repeat_interleave(hq // hkv, 0)
        V = torch.from_numpy(vo[b, :, :L]).double().repeat_interleave(hq // hkv, 0)
        Q = torch.from_numpy(q[b]).double().unsqueeze(1)
        o = torch.nn.functional.scaled_dot_product_attention(Q, K, V, scale=0.125)
        assert_allclose_ref(got[b], o[:, 0].numpy(), 1e-4, 1e-5, f"sdpa b={b}")


def test_decode_known_answers():
    rng = np.random.default_rng(7)
    hkv, bs, d, hq = 2, 16, 32, 4
    nb = 16
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d)
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    # L = 1: the output is the single V row, exactly
    t1 = np.array([[5]], np.int32)
    out = oracle.decode_attention(q, kp, vp, t1, np.int32([1]), 0.3)
    for h in range(hq):
        assert np.array_equal(out[0, h], vp[5, h // 2, 0])
    # constant keys: uniform weights -> the mean of the V rows
    kc = kp.copy()
    kc[:] = rng.standard_normal(d).astype(np.float32)
    tab = np.array([[1, 2, 3]], np.int32)
    out = oracle.decode_attention(q, kc, vp, tab, np.int32([40]), 0.2)
    pos = np.arange(40)
    mean = vp[tab[0, pos // bs], :, pos % bs, :].astype(np.float64).mean(axis=0)
    for h in range(hq):
        assert np.abs(out[0, h] - mean[h // 2]).max() < 1e-5
    # one dominating score selects that V row
    kd = np.zeros_like(kp)
    kd[2, :, 7, :] = 50.0
    qd = np.ones((1, hq, d), np.float32)
    out = oracle.decode_attention(qd, kd, vp, tab, np.int32([40]), 1.0)
    for h in range(hq):
        assert np.allclose(out[0, h], vp[2, h // 2, 7], atol=1e-6)
    # GQA: query heads of one group with equal queries give equal outputs
    qg = np.repeat(rng.standard_normal((1, hkv, 1, d)).astype(np.float32), 2, axis=2)
    out = oracle.decode_attention(qg.reshape(1, hq, d), kp, vp, tab, np.int32([40]), 0.2)
    assert np.array_equal(out[0, 0], out[0, 1]) and np.array_equal(out[0, 2], out[0, 3])
    # zero context -> zeros
    out = oracle.decode_attention(q, kp, vp, tab, np.int32([0]), 0.2)
    assert not out.any()


def test_decode_block_permutation_invariance():
    rng = np.random.default_rng(8)
    hkv, bs, d, hq, nb = 2, 16, 64, 8, 24
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d)
    ctx = np.int32([150])
    tab = make_tables(rng, ctx, bs, nb)
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    base = oracle.decode_attention(q, kp, vp, tab, ctx, 0.1)
    # move every block to a new physical id, with its data
    perm = rng.permutation(nb).astype(np.int32)
    kp2, vp2 = np.empty_like(kp), np.empty_like(vp)
    kp2[perm] = kp
    vp2[perm] = vp
    tab2 = np.where(tab >= 0, perm[np.maximum(tab, 0)], -1).astype(np.int32)
    assert np.array_equal(oracle.decode_attention(q, kp2, vp2, tab2, ctx, 0.1), base)


def test_decode_invalid_block_ids_are_left_out():
    rng = np.random.default_rng(9)
    hkv, bs, d, hq, nb = 1, 16, 32, 2, 10
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d)
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    tab = np.array([[3, 99, 5]], np.int32)  # block 99 does not exist
    got = oracle.decode_attention(q, kp, vp, tab, np.int32([40]), 0.2)
    # same as attending to tokens 0-15 and 32-39 only
    pos = np.concatenate([np.arange(16), np.arange(32, 40)])
    blk = tab[0, pos // bs]
    K = kp[blk, 0, pos % bs].astype(np.float64)
    V = vp[blk, 0, pos % bs].astype(np.float64)
    for h in range(hq):
        s = K @ q[0, h].astype(np.float64) * 0.2
        p = np.exp(s - s.max())
        assert np.abs(got[0, h] - (p / p.sum()) @ V).max() < 1e-5


@pytest.mark.parametrize("psize", [16, 48, 256, 512])
def test_splitk_merge_equals_single_pass(psize):
    rng = np.random.default_rng(10)
    hkv, bs, d, hq = 2, 16, 64, 8
    ctx = np.array([1, 31, 256, 257, 700], np.int32)
    nb = 80
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d, "bf16")
    tables = make_tables(rng, ctx, bs, nb)
    q = rng.standard_normal((len(ctx), hq, d)).astype(np.float32)
    single = oracle.decode_attention(q, kp, vp, tables, ctx, 0.125)
    split, (m, l, acc) = oracle.decode_splitk(q, kp, vp, tables, ctx, 0.125, psize)
    assert np.abs(split - single).max() < 1e-5
    # each partial is a normalised softmax piece: l >= 1 (its own max contributes e^0)
    npart = (ctx + psize - 1) // psize
    for b in range(len(ctx)):
        assert (l[b, :, :npart[b]] >= 1.0).all()


def test_multithreaded_oracle_is_identical():
    rng = np.random.default_rng(11)
    hkv, bs, d, hq = 4, 16, 128, 16
    ctx = contexts(rng, 9, 1, 300)
    nb = int(sum((c + 15) // 16 for c in ctx))
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d, "bf16")
    tables = make_tables(rng, ctx, bs, nb)
    q = rng.standard_normal((len(ctx), hq, d)).astype(np.float32)
    a = oracle.decode_attention(q, kp, vp, tables, ctx, 0.1)
    b = oracle.decode_attention(q, kp, vp, tables, ctx, 0.1, n_threads=5)
    assert np.array_equal(a, b)


# ---- causal prefill over the paged pool -------------------------------------

@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("hq,hkv,d", [(8, 2, 64), (4, 4, 32), (32, 8, 128)])
def test_prefill_vs_independent_f64(dtype, hq, hkv, d):
    from tests.helpers import make_prefill, ref_prefill_f64
    rng = np.random.default_rng(hq * 10 + d)
    bs = 16
    n_new = np.array([1, 17, 40, 0, 5], np.int32)
    ctx = n_new + np.array([0, 0, 100, 7, 33], np.int32)   # square prefills and chunked ones
    nb = int(sum((c + bs - 1) // bs for c in ctx)) + 5
    kp, vp, kf, vf = make_pool(rng, nb, hkv, bs, d, dtype)
    if dtype == "bf16":
        kf, vf = oracle.pool_as_f32(kp), oracle.pool_as_f32(vp)
    tables = make_tables(rng, ctx, bs, nb)
    qs = make_prefill(rng, n_new, ctx)
    q = rng.standard_normal((int(qs[-1]), hq, d)).astype(np.float32)
    scale = 1 / math.sqrt(d)
    got = oracle.prefill_attention(q, kp, vp, tables, qs, ctx, scale)
    want = ref_prefill_f64(q, kf, vf, tables, qs, ctx, scale)
    assert np.abs(got - want).max() < 2e-5


def test_prefill_square_case_vs_torch_causal_sdpa():
    """ctx == n (the reference's square causal prefill) against torch's
    is_causal scaled_dot_product_attention in float64."""
    from tests.helpers import make_prefill
    rng = np.random.default_rng(3)
    hq, hkv, d, bs, n = 8, 2, 64, 16, 70
    nb = 8
    kp, vp, kf, vf = make_pool(rng, nb, hkv, bs, d, "f32")
    tables = make_tables(rng, [n], bs, nb)
    qs = make_prefill(rng, [n], [n])
    q = rng.standard_normal((n, hq, d)).astype(np.float32)
    got = oracle.prefill_attention(q, kp, vp, tables, qs, [n], 0.125)
    pos = np.arange(n)
    K = torch.from_numpy(kf[tables[0, pos // bs], :, pos % bs, :]).double()  # [n, Hkv, D]
    V = torch.from_numpy(vf[tables[0, pos // bs], :, pos % bs, :]).double()
    Q = torch.from_numpy(q).double().transpose(0, 1)                          # [Hq, n, D]
    K = K.transpose(0, 1).repeat_interleave(hq // hkv, dim=0).contiguous()
    V = V.transpose(0, 1).repeat_interleave(hq // hkv, dim=0).contiguous()
    ref = torch.nn.functional.scaled_dot_product_attention(Q, K, V, is_causal=True, scale=0.125)
    assert np.abs(got - ref.transpose(0, 1).numpy()).max() < 2e-5


def test_prefill_last_token_is_decode_and_negative_positions_are_zero():
    from tests.helpers import make_prefill
    rng = np.random.default_rng(4)
    hq, hkv, d, bs = 4, 2, 32, 16
    n_new = np.array([9, 3, 1], np.int32)
    ctx = np.array([40, 3, 2], np.int32)
    nb = 10
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d, "bf16")
    tables = make_tables(rng, ctx, bs, nb)
    qs = make_prefill(rng, n_new, ctx)
    q = rng.standard_normal((int(qs[-1]), hq, d)).astype(np.float32)
    got = oracle.prefill_attention(q, kp, vp, tables, qs, ctx, 0.2)
    # the last new token of each sequence attends to its whole context: a decode row
    last = qs[1:] - 1
    dec = oracle.decode_attention(q[last], kp, vp, tables, ctx, 0.2)
    assert np.array_equal(got[last], dec)
    # more new tokens than context: the rows before position 0 are zero
    bad = oracle.prefill_attention(q, kp, vp, tables, qs, np.array([40, 1, 2], np.int32), 0.2)
    assert np.all(bad[qs[1]:qs[1] + 2] == 0.0) and np.any(bad[qs[1] + 2] != 0.0)


# ---- 1-byte KV storage (int8 / OCP fp8 e4m3 with per-row scales) ------------

def test_e4m3_decode_matches_torch_for_every_code():
    codes = np.arange(256, dtype=np.uint8)
    ours = oracle.f32_from_e4m3(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan) and nan.sum() == 2       # 0x7f, 0xff
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_e4m3_encode_matches_torch_round_to_nearest_even():
    """Within the format's range torch's cast is round-to-nearest-even; the
    encoder must give the same byte.  Sample: every representable value, every
    midpoint between neighbours (the ties), and dense random magnitudes."""
    vals = oracle.f32_from_e4m3(np.arange(256, dtype=np.uint8))
    pos = np.unique(vals[(vals >= 0) & np.isfinite(vals)])
    mids = ((pos[1:].astype(np.float64) + pos[:-1]) / 2).astype(np.float32)
    rng = np.random.default_rng(5)
    dense = (rng.random(20000) * 464).astype(np.float32) * rng.choice([-1, 1], 20000)
    tiny = (rng.random(2000) * 2 ** -5).astype(np.float32)
    x = np.concatenate([pos, -pos, mids, -mids, dense, tiny, [464.0, -464.0, 0.0]]).astype(np.float32)
    ours = oracle.e4m3_from_f32(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_e4m3_encode_saturates_and_keeps_nan():
    x = np.array([465.0, 480.0, 1e6, np.inf, -500.0, -np.inf, np.nan], np.float32)
    assert oracle.e4m3_from_f32(x).tolist() == [0x7e, 0x7e, 0x7e, 0x7e, 0xfe, 0xfe, 0x7f]


def test_int8_rows_match_independent_numpy_formulation():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((300, 128)) * rng.random((300, 1)) * 10).astype(np.float32)
    x[0] = 0.0                                   # all-zero row: scale 0, bytes 0
    x[1, :] = np.float32(0.5) * np.arange(128) / 127.0   # exact ties of rint
    q, s = oracle.quantize_rows(x, oracle.I8)
    amax = np.abs(x).max(axis=1)
    inv = np.where(amax > 0, np.float32(127.0) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
    want = np.clip(np.rint(x * inv[:, None]), -127, 127).astype(np.int8)
    assert np.array_equal(q.view(np.int8), want)
    assert np.array_equal(s, (amax / np.float32(127.0)).astype(np.float32))
    deq = oracle.dequantize_pool(q, s, oracle.I8)
    assert np.all(np.abs(deq - x) <= s[:, None] * 0.5 * (1 + 1e-5) + 1e-30)


def test_fp8_rows_match_torch_cast_of_the_scaled_row():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((300, 64)) * 3).astype(np.float32)
    q, s = oracle.quantize_rows(x, oracle.FP8)
    amax = np.abs(x).max(axis=1)
    inv = (np.float32(448.0) / amax).astype(np.float32)
    ref = torch.from_numpy((x * inv[:, None]).astype(np.float32)).to(torch.float8_e4m3fn)
    assert np.array_equal(q, ref.view(torch.uint8).numpy())
    assert np.array_equal(s, (amax / np.float32(448.0)).astype(np.float32))
    deq = oracle.dequantize_pool(q, s, oracle.FP8)
    assert np.all(np.abs(deq - x) <= np.abs(x) * 2.0 ** -4 + s[:, None] * 2.0 ** -9 + 1e-30)


@pytest.mark.parametrize("dtype", ["i8", "fp8"])
def test_append_q_matches_fancy_indexing(dtype):
    code = oracle.I8 if dtype == "i8" else oracle.FP8
    rng = np.random.default_rng(8)
    nb, hkv, bs, d, n = 20, 4, 16, 64, 150
    kp = rng.integers(0, 256, (nb, hkv, bs, d), dtype=np.uint8)   # canary bytes
    vp = kp.copy()
    ks = np.full((nb, hkv, bs), 7.0, np.float32)
    vs = ks.copy()
    slots = rng.permutation(nb * bs)[:n].astype(np.int64)
    slots[::13] = -1
    kn = rng.standard_normal((n, hkv, d)).astype(np.float32)
    vn = rng.standard_normal((n, hkv, d)).astype(np.float32)
    ek, ev, eks, evs = kp.copy(), vp.copy(), ks.copy(), vs.copy()
    oracle.append_q(kp, vp, ks, vs, kn, vn, slots, code)
    ok = slots >= 0
    blk, row = slots[ok] // bs, slots[ok] % bs
    qk, sk = oracle.quantize_rows(kn[ok].reshape(-1, d), code)
    qv, sv = oracle.quantize_rows(vn[ok].reshape(-1, d), code)
    ek[blk, :, row, :] = qk.reshape(-1, hkv, d)
    ev[blk, :, row, :] = qv.reshape(-1, hkv, d)
    eks[blk, :, row] = sk.reshape(-1, hkv)
    evs[blk, :, row] = sv.reshape(-1, hkv)
    assert np.array_equal(kp, ek) and np.array_equal(vp, ev)
    assert np.array_equal(ks, eks) and np.array_equal(vs, evs)
