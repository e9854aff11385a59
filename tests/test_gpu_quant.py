"""GPU parity of the 1-byte KV pools (int8 and OCP fp8 e4m3, one fp32 scale
per (token, KV head) row) against the oracle.

  * append_q: bytes and scales bit-exact (the oracle quantizes with the same
    rules: tests/test_oracle.py pins them against torch's e4m3 cast and an
    independent numpy int8 formulation);
  * gather_q: dequantized values bit-exact (byte value * row scale);
  * decode_attention_q: within max-abs 1e-4 / rel 1e-3 of the oracle's decode
    on the dequantized fp32 pool (the decode tolerance).
"""
import math

import numpy as np
import pytest
import torch

import oracle
from rustral_amd import kv
from tests.gpu_util import say, to_dev, to_np
from tests.helpers import assert_allclose_ref, contexts, make_tables

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4
CODE = {"int8": oracle.I8, "fp8": oracle.FP8}


def quant_case(seed, nb, hkv, bs, d, fmt, fill_slots=None):
    """Pools filled through the oracle's quantizing append: every slot (or the
    given ones) holds a quantized N(0,1) row; other rows keep canary bytes and
    scale 1e30 (never read for valid tokens)."""
    rng = np.random.default_rng(seed)
    kp = rng.integers(0, 256, (nb, hkv, bs, d), dtype=np.uint8)
    vp = rng.integers(0, 256, (nb, hkv, bs, d), dtype=np.uint8)
    ks = np.full((nb, hkv, bs), 1e30, np.float32)
    vs = ks.copy()
    slots = np.arange(nb * bs, dtype=np.int64) if fill_slots is None else fill_slots
    kn = (rng.standard_normal((len(slots), hkv, d)) * rng.random((len(slots), hkv, 1)) * 3)
    vn = rng.standard_normal((len(slots), hkv, d))
    oracle.append_q(kp, vp, ks, vs, kn.astype(np.float32), vn.astype(np.float32), slots,
                    CODE[fmt])
    return kp, vp, ks, vs


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
@pytest.mark.parametrize("hkv,d,nl", [(8, 128, 1), (4, 64, 3), (2, 32, 2), (32, 128, 1)])
def test_append_q_bitexact(dev, fmt, hkv, d, nl):
    say(f"append_q fmt={fmt} hkv={hkv} d={d} layers={nl}")
    rng = np.random.default_rng(hkv * 100 + d + nl)
    nb, bs, n = 40, 16, 300
    kp = rng.integers(0, 256, (nl, nb, hkv, bs, d), dtype=np.uint8)
    vp = rng.integers(0, 256, (nl, nb, hkv, bs, d), dtype=np.uint8)
    ks = rng.standard_normal((nl, nb, hkv, bs)).astype(np.float32)
    vs = rng.standard_normal((nl, nb, hkv, bs)).astype(np.float32)
    slots = rng.permutation(nb * bs)[:n].astype(np.int64)
    slots[::29] = -1
    kn = (rng.standard_normal((nl, n, hkv, d)) * 4).astype(np.float32)
    vn = rng.standard_normal((nl, n, hkv, d)).astype(np.float32)
    kn[0, 3] = 0.0                     # an all-zero row: scale 0, bytes 0
    kn[0, 4, 0, 5] = 1e4               # one dominating element
    g = [to_dev(a, dev) for a in (kp, vp, ks, vs)]
    if nl == 1:
        kv.append_q(g[0][0], g[1][0], g[2][0], g[3][0], to_dev(kn[0], dev), to_dev(vn[0], dev),
                    to_dev(slots, dev), fmt)
    else:
        kv.append_q(*g, to_dev(kn, dev), to_dev(vn, dev), to_dev(slots, dev), fmt)
    for l in range(nl):
        oracle.append_q(kp[l], vp[l], ks[l], vs[l], kn[l], vn[l], slots, CODE[fmt])
    torch.cuda.synchronize()
    assert np.array_equal(to_np(g[0]), kp) and np.array_equal(to_np(g[1]), vp)
    assert np.array_equal(to_np(g[2]).view(np.uint32), ks.view(np.uint32))
    assert np.array_equal(to_np(g[3]).view(np.uint32), vs.view(np.uint32))


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_gather_q_dequantizes_bitexact(dev, fmt):
    say(f"gather_q fmt={fmt}")
    rng = np.random.default_rng(21)
    nb, hkv, bs, d = 120, 8, 16, 128
    ctx = np.array([0, 1, 15, 16, 17, 300, 999], np.int32)
    kp, vp, ks, vs = quant_case(21, nb, hkv, bs, d, fmt)
    tables = make_tables(rng, ctx, bs, nb)
    k_out, v_out = kv.gather_q(to_dev(kp, dev), to_dev(vp, dev), to_dev(ks, dev),
                               to_dev(vs, dev), to_dev(tables, dev), to_dev(ctx, dev), fmt,
                               max_ctx=1008)
    torch.cuda.synchronize()
    kf = oracle.dequantize_pool(kp, ks, CODE[fmt])
    vf = oracle.dequantize_pool(vp, vs, CODE[fmt])
    wk, wv = oracle.gather(kf, vf, tables, ctx, max_ctx=1008)
    assert np.array_equal(to_np(k_out), wk) and np.array_equal(to_np(v_out), wv)


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
@pytest.mark.parametrize("bs,d", [(12, 32), (16, 64), (8, 128)])
def test_gather_q_every_byte_code_and_block_sizes(dev, fmt, bs, d):
    """Every one of the 256 byte codes (fp8: NaN codes 0x7f / 0xff, both
    zeros, subnormals, +-448) at several scales, block sizes that are not a
    power of two, partial last blocks: the dequantized values equal the
    oracle's bit for bit (NaNs compared as bit patterns)."""
    say(f"gather_q all codes fmt={fmt} bs={bs} d={d}")
    rng = np.random.default_rng(29)
    hkv, nb = 3, 40
    kp = (np.arange(nb * hkv * bs * d) % 256).astype(np.uint8).reshape(nb, hkv, bs, d)
    vp = np.roll(kp, 7, axis=-1).copy()
    ks = rng.choice(np.array([1.0, 0.5, 3.0e-3, 17.25, 2.0 ** -20], np.float32),
                    (nb, hkv, bs)).astype(np.float32)
    vs = rng.random((nb, hkv, bs)).astype(np.float32)
    ctx = np.array([bs * 5 + 3, 1, bs, 0, bs * 9], np.int32)
    tables = make_tables(rng, ctx, bs, nb)
    k_out, v_out = kv.gather_q(to_dev(kp, dev), to_dev(vp, dev), to_dev(ks, dev),
                               to_dev(vs, dev), to_dev(tables, dev), to_dev(ctx, dev), fmt,
                               max_ctx=int(ctx.max()))
    torch.cuda.synchronize()
    kf = oracle.dequantize_pool(kp, ks, CODE[fmt])
    vf = oracle.dequantize_pool(vp, vs, CODE[fmt])
    wk, wv = oracle.gather(kf, vf, tables, ctx, max_ctx=int(ctx.max()), out_f32=True)
    assert np.array_equal(to_np(k_out).view(np.uint32), wk.view(np.uint32))
    assert np.array_equal(to_np(v_out).view(np.uint32), wv.view(np.uint32))


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_gather_q_packed_layout_bitexact(dev, fmt):
    """The packed KVCache layout (sequence b's [Hkv, L_b, D] at its offset):
    dequantized values equal the oracle's gather of the dequantized pool, and
    the guard rows between sequences and after the last stay untouched."""
    say(f"gather_q packed fmt={fmt}")
    rng = np.random.default_rng(23)
    nb, hkv, bs, d = 96, 4, 16, 64
    ctx = np.array([5, 0, 16, 33, 250, 1], np.int32)
    kp, vp, ks, vs = quant_case(23, nb, hkv, bs, d, fmt)
    tables = make_tables(rng, ctx, bs, nb)
    gap = hkv * d  # one row of guard elements after every sequence
    sizes = ctx.astype(np.int64) * hkv * d + gap
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    total = int(sizes.sum())
    guard = np.float32(-7.25)
    k_out = torch.full((total,), float(guard), dtype=torch.float32, device=dev)
    v_out = torch.full((total,), float(guard), dtype=torch.float32, device=dev)
    kv.gather_q(to_dev(kp, dev), to_dev(vp, dev), to_dev(ks, dev), to_dev(vs, dev),
                to_dev(tables, dev), to_dev(ctx, dev), fmt, out_offsets=to_dev(offs, dev),
                out_total=total, k_out=k_out, v_out=v_out)
    torch.cuda.synchronize()
    kf = oracle.dequantize_pool(kp, ks, CODE[fmt])
    vf = oracle.dequantize_pool(vp, vs, CODE[fmt])
    wk = np.full(total, guard, np.float32)
    wv = np.full(total, guard, np.float32)
    oracle.gather(kf, vf, tables, ctx, out_offsets=offs, out_f32=True, k_out=wk, v_out=wv)
    assert np.array_equal(to_np(k_out), wk) and np.array_equal(to_np(v_out), wv)
    for b in range(len(ctx)):   # the guard rows themselves
        g0 = int(offs[b] + ctx[b] * hkv * d)
        assert (wk[g0:g0 + gap] == guard).all()


def run_q(dev, q, kp, vp, ks, vs, tables, ctx, scale, fmt, max_context=None):
    out = kv.decode_attention_q(to_dev(q, dev), to_dev(kp, dev), to_dev(vp, dev),
                                to_dev(ks, dev), to_dev(vs, dev), to_dev(tables, dev),
                                to_dev(ctx, dev), scale, fmt, max_context=max_context)
    torch.cuda.synchronize()
    return to_np(out)


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 2, 64), (16, 2, 128), (8, 1, 128),
                                      (4, 4, 64), (2, 1, 64), (2, 2, 128), (4, 2, 128),
                                      (16, 2, 64)])
def test_decode_q_matches_oracle_on_dequantized_pool(dev, fmt, hq, hkv, d):
    say(f"decode_q fmt={fmt} hq={hq} hkv={hkv} d={d}")
    rng = np.random.default_rng(hq * 7 + d)
    ctx = np.array([1, 2, 15, 16, 17, 255, 512, 513, 1000, 2100], np.int32)
    bs = 16
    nb = int(sum((c + bs - 1) // bs for c in ctx)) + 4
    kp, vp, ks, vs = quant_case(hq + d, nb, hkv, bs, d, fmt)
    tables = make_tables(rng, ctx, bs, nb)
    q = rng.standard_normal((len(ctx), hq, d)).astype(np.float32)
    scale = float(np.float32(1 / math.sqrt(d)))
    got = run_q(dev, q, kp, vp, ks, vs, tables, ctx, scale, fmt)
    kf = oracle.dequantize_pool(kp, ks, CODE[fmt])
    vf = oracle.dequantize_pool(vp, vs, CODE[fmt])
    want = oracle.decode_attention(q, kf, vf, tables, ctx, scale)
    assert_allclose_ref(got, want, RTOL, ATOL, "gpu vs oracle (dequantized pool)")


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_decode_q_config2_shape_and_partial_blocks(dev, fmt):
    """configs[2] shape (B64, Hq32, Hkv8, D128, L in U[512, 4096]); only the
    context's slots are written, so the unwritten rows of each sequence's last
    block keep canary bytes and a 1e30 scale and must not leak in."""
    say(f"decode_q configs[2] shape fmt={fmt}")
    rng = np.random.default_rng(30)
    ctx = contexts(rng, 64, 512, 4096)
    bs, hkv, d = 16, 8, 128
    nb = int(sum((c + bs - 1) // bs for c in ctx))
    tables = make_tables(rng, ctx, bs, nb)
    slots = np.concatenate([tables[b, np.arange(L) // bs].astype(np.int64) * bs + np.arange(L) % bs
                            for b, L in enumerate(ctx)])
    kp, vp, ks, vs = quant_case(31, nb, hkv, bs, d, fmt, fill_slots=slots)
    q = rng.standard_normal((64, 32, d)).astype(np.float32)
    got = run_q(dev, q, kp, vp, ks, vs, tables, ctx, 1 / math.sqrt(d), fmt, max_context=4096)
    kf = oracle.dequantize_pool(kp, ks, CODE[fmt])
    vf = oracle.dequantize_pool(vp, vs, CODE[fmt])
    want = oracle.decode_attention(q, kf, vf, tables, ctx, 1 / math.sqrt(d), n_threads=8)
    assert np.isfinite(got).all()
    assert_allclose_ref(got, want, RTOL, ATOL, "gpu vs oracle")


@pytest.mark.parametrize("hq,hkv", [(32, 8), (8, 4), (4, 4)])
def test_decode_q_int8_wide_dynamic_range(dev, hq, hkv):
    """int8 pools with K rows scaled by 10^U(-1.5, 1.5) and V rows by
    10^U(-2, 2) per (token, head), q heads by 10^U(-1.5, 1), one q head all
    zeros and one a single spike over 1e-3 values.  For G <= 4 the kernel
    runs QK^T and PV on the integer matrix cores with q and the PV weights in
    four int8 limbs, fixed point against each head's maximum: these inputs
    put the small terms many decades under that maximum, where a dropped or
    mis-scaled limb would show.  (G = 8 runs the bf16 path, q as bf16 hi +
    lo; the other cases cover it.)"""
    say(f"decode_q int8 wide range hq={hq} hkv={hkv}")
    rng = np.random.default_rng(5 + hq)
    ctx = np.array([1, 17, 300, 640, 641, 1500, 2600], np.int32)
    bs, d = 16, 128
    nb = int(sum((c + bs - 1) // bs for c in ctx)) + 4
    n = nb * bs
    kn = rng.standard_normal((n, hkv, d)) * 10 ** rng.uniform(-1.5, 1.5, (n, hkv, 1))
    vn = rng.standard_normal((n, hkv, d)) * 10 ** rng.uniform(-2, 2, (n, hkv, 1))
    kp = np.zeros((nb, hkv, bs, d), np.uint8)
    vp = np.zeros_like(kp)
    ks = np.zeros((nb, hkv, bs), np.float32)
    vs = np.zeros_like(ks)
    oracle.append_q(kp, vp, ks, vs, kn.astype(np.float32), vn.astype(np.float32),
                    np.arange(n, dtype=np.int64), oracle.I8)
    tables = make_tables(rng, ctx, bs, nb)
    q = rng.standard_normal((len(ctx), hq, d)) * 10 ** rng.uniform(-1.5, 1, (len(ctx), hq, 1))
    q = q.astype(np.float32)
    q[0, 0] = 0.0
    q[1, 1] = 1e-3
    q[1, 1, 5] = 50.0
    scale = float(np.float32(1 / math.sqrt(d)))
    got = run_q(dev, q, kp, vp, ks, vs, tables, ctx, scale, "int8")
    want = oracle.decode_attention(q, oracle.dequantize_pool(kp, ks, oracle.I8),
                                   oracle.dequantize_pool(vp, vs, oracle.I8), tables, ctx, scale)
    assert_allclose_ref(got, want, RTOL, ATOL, "int8 wide range vs oracle")


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_decode_q_invalid_blocks_empty_sequences_and_clamp(dev, fmt):
    """1-byte pools over 70 sequences (more than one 64-length scan of the
    work plan): block ids of -1 and past the pool leave their tokens out,
    empty sequences give zero rows, a context past its table is clamped to
    the table, and a second call gives the same bits."""
    say(f"decode_q invalid ids / empty / clamp fmt={fmt}")
    rng = np.random.default_rng(11)
    hkv, bs, d, hq, mb = 8, 16, 128, 32, 96
    ctx = rng.integers(0, 1500, size=70).astype(np.int32)
    ctx[::9] = 0
    ctx[4] = 1
    ctx[1] = 5000                                   # > mb * bs: clamped to 1536
    eff = np.minimum(ctx, mb * bs)
    nb = int(sum((c + bs - 1) // bs for c in eff)) + 8
    kp, vp, ks, vs = quant_case(12, nb, hkv, bs, d, fmt)
    tables = make_tables(rng, eff, bs, nb, max_blocks=mb)
    seq = int(np.argmax(eff >= 6 * bs))
    tables[seq, 3] = -1
    tables[seq, 5] = 10 ** 6
    q = rng.standard_normal((len(ctx), hq, d)).astype(np.float32)
    scale = float(np.float32(1 / math.sqrt(d)))
    got = run_q(dev, q, kp, vp, ks, vs, tables, ctx, scale, fmt)
    want = oracle.decode_attention(q, oracle.dequantize_pool(kp, ks, CODE[fmt]),
                                   oracle.dequantize_pool(vp, vs, CODE[fmt]), tables, ctx, scale,
                                   n_threads=8)
    assert_allclose_ref(got, want, RTOL, ATOL, "1-byte invalid ids / clamp vs oracle")
    assert not got[ctx == 0].any()
    again = run_q(dev, q, kp, vp, ks, vs, tables, ctx, scale, fmt)
    assert np.array_equal(got, again)


def test_decode_q_quantization_error_is_small(dev):
    """Against fp32 attention on the unquantized values: the int8 / fp8
    storage error stays within a few 1e-2 (max-abs) on N(0,1) data."""
    say("decode_q vs unquantized fp32")
    rng = np.random.default_rng(40)
    ctx = np.array([300, 1000, 2000], np.int32)
    bs, hkv, d, hq = 16, 2, 128, 8
    nb = int(sum((c + bs - 1) // bs for c in ctx))
    tables = make_tables(rng, ctx, bs, nb)
    kf = rng.standard_normal((nb, hkv, bs, d)).astype(np.float32)
    vf = rng.standard_normal((nb, hkv, bs, d)).astype(np.float32)
    q = rng.standard_normal((3, hq, d)).astype(np.float32)
    want = oracle.decode_attention(q, kf, vf, tables, ctx, 1 / math.sqrt(d))
    slots = np.arange(nb * bs, dtype=np.int64)
    for fmt, tol in (("int8", 2e-2), ("fp8", 6e-2)):
        kp = np.zeros((nb, hkv, bs, d), np.uint8)
        vp = np.zeros_like(kp)
        ks = np.zeros((nb, hkv, bs), np.float32)
        vs = np.zeros_like(ks)
        oracle.append_q(kp, vp, ks, vs, kf.transpose(0, 2, 1, 3).reshape(-1, hkv, d),
                        vf.transpose(0, 2, 1, 3).reshape(-1, hkv, d), slots, CODE[fmt])
        got = run_q(dev, q, kp, vp, ks, vs, tables, ctx, 1 / math.sqrt(d), fmt)
        err = np.abs(got - want).max()
        say(f"{fmt}: max |decode_q - fp32 decode| = {err:.3e}")
        assert err < tol


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
@pytest.mark.parametrize("P", [128, 384, 512, 576])
def test_decode_q_caller_partition_sizes(dev, fmt, P):
    """1-byte pools at requested partition sizes (the smallest of the 512- and
    640-token builds that holds the size, the slots past it masked), against
    the oracle on the dequantized pool."""
    say(f"decode_q partition_size={P} fmt={fmt}")
    rng = np.random.default_rng(P)
    ctx = np.array([1, 100, 128, 129, 384, 385, 1000, 2500], np.int32)
    nb, hkv, bs, d = 360, 8, 16, 128
    kp, vp, ks, vs = quant_case(P, nb, hkv, bs, d, fmt)
    tables = make_tables(rng, ctx, bs, nb)
    q = rng.standard_normal((len(ctx), 32, d)).astype(np.float32)
    scale = float(np.float32(1.0 / math.sqrt(d)))
    out = kv.decode_attention_q(to_dev(q, dev), to_dev(kp, dev), to_dev(vp, dev), to_dev(ks, dev),
                                to_dev(vs, dev), to_dev(tables, dev), to_dev(ctx, dev), scale, fmt,
                                partition_size=P)
    torch.cuda.synchronize()
    want = oracle.decode_attention(q, oracle.dequantize_pool(kp, ks, CODE[fmt]),
                                   oracle.dequantize_pool(vp, vs, CODE[fmt]), tables, ctx, scale)
    assert_allclose_ref(to_np(out), want, RTOL, ATOL, f"1-byte partition {P} vs oracle")


@pytest.mark.parametrize("P", [0, 256, 640])
@pytest.mark.parametrize("max_context", [None, 1000])
@pytest.mark.parametrize("fmt", ["int8", "fp8"])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 2, 64), (8, 1, 128), (16, 2, 64),
                                      (8, 8, 128), (16, 8, 64)])
def test_decode_append_q_fused_matches_append_q_then_decode_q(dev, P, max_context, fmt, hq,
                                                              hkv, d):
    """rkv_decode_attention_append_q == rkv_append_q of the new rows followed
    by rkv_decode_attention_q, bit for bit in the byte pools, the scale pools
    and the output: new tokens at the first, middle and last row of a block
    and at partition boundaries, an all-zero row (scale 0), a row with a
    large value (fp8 saturation range), invalid block ids (-1 and past the
    pool: nothing written), an empty sequence, and lengths clamped by
    max_context 1000 (their rows not written); every G the kernels build
    (1, 2, 4, 8).  The output is also checked against the oracle on the
    dequantized appended pools, over the lengths clamped to max_context."""
    bs = 16
    ctx = np.array([1, 2, 16, 17, 640, 641, 1281, 0, 40, 50, 33, 256], np.int32)
    say(f"decode append_q fused fmt={fmt} P={P} hq={hq} hkv={hkv} d={d} max_context={max_context}")
    rng = np.random.default_rng(11 * P + hq + d)
    nb = int(sum((int(c) + bs - 1) // bs for c in ctx)) + 3
    kp, vp, ks, vs = quant_case(hq + d + P, nb, hkv, bs, d, fmt)
    tables = make_tables(rng, ctx, bs, nb)
    tables[8, (40 - 1) // bs] = -1
    tables[9, (50 - 1) // bs] = nb + 3
    kn = (rng.standard_normal((len(ctx), hkv, d)) * 2).astype(np.float32)
    vn = rng.standard_normal((len(ctx), hkv, d)).astype(np.float32)
    kn[10] = 0.0                      # scale 0
    vn[11, :, 3] = 5e4                # one large element
    cap = min(max_context if max_context is not None else 1 << 30, tables.shape[1] * bs)
    slots = np.full(len(ctx), -1, np.int64)
    for b, L in enumerate(ctx):
        if 0 < L <= cap:
            blk = int(tables[b, (L - 1) // bs])
            slots[b] = blk * bs + (L - 1) % bs if 0 <= blk < nb else -1
    q = rng.standard_normal((len(ctx), hq, d)).astype(np.float32)
    scale = float(np.float32(1.0 / math.sqrt(d)))
    qd, td, cd = to_dev(q, dev), to_dev(tables, dev), to_dev(ctx, dev)
    knd, vnd = to_dev(kn, dev), to_dev(vn, dev)
    k1, v1, s1, t1 = to_dev(kp, dev), to_dev(vp, dev), to_dev(ks, dev), to_dev(vs, dev)
    k2, v2, s2, t2 = k1.clone(), v1.clone(), s1.clone(), t1.clone()
    kv.append_q(k1, v1, s1, t1, knd, vnd, to_dev(slots, dev), fmt)
    want = kv.decode_attention_q(qd, k1, v1, s1, t1, td, cd, scale, fmt,
                                 max_context=max_context, partition_size=P)
    got = kv.decode_attention_append_q(qd, k2, v2, s2, t2, knd, vnd, td, cd, scale, fmt,
                                       max_context=max_context, partition_size=P)
    torch.cuda.synchronize()
    assert torch.equal(k2, k1) and torch.equal(v2, v1), "byte pools differ"
    assert torch.equal(s2.view(torch.int32), s1.view(torch.int32)), "K scales differ"
    assert torch.equal(t2.view(torch.int32), t1.view(torch.int32)), "V scales differ"
    assert torch.equal(got.view(torch.int32), want.view(torch.int32)), \
        f"max diff {(got - want).abs().max().item()}"
    ref = oracle.decode_attention(q, oracle.dequantize_pool(to_np(k1), to_np(s1), CODE[fmt]),
                                  oracle.dequantize_pool(to_np(v1), to_np(t1), CODE[fmt]), tables,
                                  np.minimum(ctx, cap), scale)
    assert_allclose_ref(to_np(got), ref, RTOL, ATOL, "fused 1-byte append vs oracle")
