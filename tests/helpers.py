"""Seeded synthetic inputs shared by the CPU and GPU tests (numpy side)."""
from __future__ import annotations

import numpy as np

import oracle


def make_pool(rng, num_blocks, hkv, bs, d, dtype="f32", canary=None):
    """K/V pools [num_blocks, Hkv, BS, D] with N(0,1) values (float32, or uint16
    bf16 bits obtained by RNE rounding)."""
    k = rng.standard_normal((num_blocks, hkv, bs, d), dtype=np.float32)
    v = rng.standard_normal((num_blocks, hkv, bs, d), dtype=np.float32)
    if canary is not None:
        k[:] = canary
        v[:] = canary
    if dtype == "bf16":
        return oracle.bf16_from_f32(k), oracle.bf16_from_f32(v), k, v
    return k, v, k, v


def make_tables(rng, ctx_lens, bs, num_blocks, max_blocks=None):
    """Block tables from a random permutation of the pool (Fisher-Yates via
    numpy), each sequence taking ceil(L/bs) distinct blocks; unused entries -1."""
    need = [(int(L) + bs - 1) // bs for L in ctx_lens]
    mbs = max(1, max(need) if max_blocks is None else max_blocks)
    assert sum(need) <= num_blocks, "pool too small"
    perm = rng.permutation(num_blocks).astype(np.int32)
    tables = np.full((len(ctx_lens), mbs), -1, dtype=np.int32)
    o = 0
    for b, n in enumerate(need):
        tables[b, :n] = perm[o:o + n]
        o += n
    return tables


def contexts(rng, n, lo, hi):
    return rng.integers(lo, hi + 1, size=n).astype(np.int32)


def ref_decode_f64(q, k_pool_f32, v_pool_f32, tables, ctx_lens, scale):
    """Independent float64 formulation (numpy gather + einsum + softmax) used
    to pin the oracle; not the oracle's loop order."""
    B, hq, d = q.shape
    nb, hkv, bs, _ = k_pool_f32.shape
    g = hq // hkv
    out = np.zeros((B, hq, d), np.float64)
    for b in range(B):
        L = int(ctx_lens[b])
        if L <= 0:
            continue
        pos = np.arange(L)
        blk = tables[b, pos // bs]
        K = k_pool_f32[blk, :, pos % bs, :].astype(np.float64)  # [L, Hkv, D]
        V = v_pool_f32[blk, :, pos % bs, :].astype(np.float64)
        qh = q[b].astype(np.float64).reshape(hkv, g, d)
        s = np.einsum("kgd,lkd->kgl", qh, K) * scale
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        out[b] = np.einsum("kgl,lkd->kgd", p, V).reshape(hq, d)
    return out


def assert_allclose_ref(got, want, rtol, atol, name=""):
    """The reference's acceptance rule (crates/core/tests/common/numeric.rs:42-66):
    pass when |d| <= atol or |d| <= rtol * max(|a|, |b|), all values finite."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{name}: shape {got.shape} vs {want.shape}"
    assert np.isfinite(got).all() and np.isfinite(want).all(), f"{name}: non-finite values"
    diff = np.abs(got - want)
    ok = (diff <= atol) | (diff <= rtol * np.maximum(np.abs(got), np.abs(want)))
    if not ok.all():
        i = np.unravel_index(np.argmax(np.where(ok, 0, diff)), diff.shape)
        raise AssertionError(f"{name}: mismatch at {i}: got {got[i]} want {want[i]} "
                             f"(max abs diff {diff.max():.3e}, rtol {rtol}, atol {atol})")


def ref_prefill_f64(q, k_pool_f32, v_pool_f32, tables, q_start, ctx_lens, scale):
    """Independent float64 formulation of causal prefill: per sequence, the
    full score matrix Q K^T * scale plus the reference's additive -1e9 mask
    above the diagonal (causal_mask_tape), a row softmax, then W V.  Rows
    whose position is negative are zero."""
    total, hq, d = q.shape
    nb, hkv, bs, _ = k_pool_f32.shape
    g = hq // hkv
    out = np.zeros((total, hq, d), np.float64)
    for b in range(len(ctx_lens)):
        s0, n, L = int(q_start[b]), int(q_start[b + 1] - q_start[b]), int(ctx_lens[b])
        if n <= 0 or L <= 0:
            continue
        pos = np.arange(L)
        blk = tables[b, pos // bs]
        K = k_pool_f32[blk, :, pos % bs, :].astype(np.float64)  # [L, Hkv, D]
        V = v_pool_f32[blk, :, pos % bs, :].astype(np.float64)
        qpos = L - n + np.arange(n)                              # position of each new token
        mask = np.where(pos[None, :] > qpos[:, None], -1e9, 0.0)  # [n, L]
        Q = q[s0:s0 + n].astype(np.float64).reshape(n, hkv, g, d)
        s = np.einsum("nkgd,lkd->nkgl", Q, K) * scale + mask[:, None, None, :]
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        o = np.einsum("nkgl,lkd->nkgd", p, V).reshape(n, hq, d)
        o[qpos < 0] = 0.0
        out[s0:s0 + n] = o
    return out


def make_prefill(rng, n_new, ctx_lens):
    """q_start offsets for sequences with n_new[b] new tokens."""
    q_start = np.zeros(len(n_new) + 1, np.int32)
    q_start[1:] = np.cumsum(n_new)
    return q_start
