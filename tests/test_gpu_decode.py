"""GPU parity of paged decode attention against the oracle.

Tolerances (from the task's parity bar):
  * fp32 pool: max-abs 1e-4 / rel 1e-3 against the fp32 oracle on the same pool;
  * bf16 pool, fp32 accumulation: the same 1e-4 / 1e-3 against the oracle run
    on the same bf16 pool, and max-abs 2e-2 against the fp32 oracle run on the
    unrounded fp32 values.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from rustral_amd import kv
from tests.gpu_util import device_case, say, to_dev, to_np
from tests.helpers import assert_allclose_ref, contexts, make_pool, make_tables

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4
BF16_VS_F32_ATOL = 2e-2


def run_gpu(dev, q, kp, vp, tables, ctx, scale, max_context=None):
    out = kv.decode_attention(to_dev(q, dev), to_dev(kp, dev), to_dev(vp, dev),
                              to_dev(tables, dev), to_dev(ctx, dev), scale,
                              max_context=max_context)
    torch.cuda.synchronize()
    return to_np(out)


def case(seed, B, hq, hkv, d, ctx, dtype, extra_blocks=3):
    rng = np.random.default_rng(seed)
    bs = 16
    nb = int(sum((int(c) + bs - 1) // bs for c in ctx)) + extra_blocks
    kp, vp, kf, vf = make_pool(rng, nb, hkv, bs, d, dtype)
    tables = make_tables(rng, ctx, bs, nb)
    q = rng.standard_normal((B, hq, d)).astype(np.float32)
    return q, kp, vp, kf, vf, tables


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("hq,hkv,d", [(4, 4, 32), (8, 4, 64), (32, 8, 128), (8, 1, 128),
                                      (16, 2, 64), (4, 2, 32)])
def test_decode_small_shapes(dev, dtype, hq, hkv, d):
    ctx = np.array([1, 2, 15, 16, 17, 31, 255, 256, 257, 600, 1000], np.int32)
    say(f"decode small dtype={dtype} hq={hq} hkv={hkv} d={d}")
    q, kp, vp, kf, vf, tables = case(hq * 1000 + d, len(ctx), hq, hkv, d, ctx, dtype)
    scale = float(np.float32(1.0 / math.sqrt(d)))
    got = run_gpu(dev, q, kp, vp, tables, ctx, scale)
    want = oracle.decode_attention(q, kp, vp, tables, ctx, scale)
    assert_allclose_ref(got, want, RTOL, ATOL, "gpu vs oracle (same pool)")
    if dtype == "bf16":
        want32 = oracle.decode_attention(q, kf, vf, tables, ctx, scale)
        assert np.abs(got - want32).max() <= BF16_VS_F32_ATOL


@pytest.mark.parametrize("g", [1, 2, 4, 8])
@pytest.mark.parametrize("d", [32, 64, 128])
def test_decode_bf16_every_group_and_head_dim(dev, g, d):
    """Every (G, D) instantiation of the bf16 kernel (QK^T and PV on the
    matrix cores, V tiles through LDS): ragged contexts, a sequence spanning
    several partitions and one short of a block, against the oracle on the
    same pool."""
    hkv = 2
    ctx = np.array([1, 16, 47, 513, 1500, 2049], np.int32)
    say(f"decode bf16 grid g={g} d={d}")
    q, kp, vp, kf, vf, tables = case(g * 100 + d, len(ctx), g * hkv, hkv, d, ctx, "bf16")
    scale = float(np.float32(1.0 / math.sqrt(d)))
    got = run_gpu(dev, q, kp, vp, tables, ctx, scale)
    want = oracle.decode_attention(q, kp, vp, tables, ctx, scale)
    assert_allclose_ref(got, want, RTOL, ATOL, "gpu vs oracle (same pool)")


def test_decode_matches_committed_golden(dev):
    import os
    say("decode golden fixture")
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "decode_small.npz"))
    got = run_gpu(dev, g["q"], g["k_pool"], g["v_pool"], g["tables"], g["ctx_lens"],
                  float(g["scale"]))
    assert_allclose_ref(got, g["expected"], RTOL, ATOL, "gpu vs golden")


def test_decode_known_answers(dev):
    say("decode known answers")
    rng = np.random.default_rng(5)
    hkv, bs, d, hq, nb = 2, 16, 128, 8, 40
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d, "bf16")
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    # L = 1 -> exactly the V row
    out = run_gpu(dev, q, kp, vp, np.array([[9]], np.int32), np.int32([1]), 0.3)
    vrow = oracle.f32_from_bf16(vp[9, :, 0])
    for h in range(hq):
        assert np.array_equal(out[0, h], vrow[h // 4])
    # zero and negative context -> zeros
    out = run_gpu(dev, np.stack([q[0], q[0]]), kp, vp, np.array([[1], [2]], np.int32),
                  np.int32([0, -3]), 0.3)
    assert not out.any()
    # GQA group with identical queries -> identical rows
    qg = np.repeat(rng.standard_normal((1, hkv, 1, d)).astype(np.float32), 4, axis=2)
    tab = make_tables(rng, np.int32([500]), bs, nb)
    out = run_gpu(dev, qg.reshape(1, hq, d), kp, vp, tab, np.int32([500]), 0.1)
    for h in range(hq):
        assert np.array_equal(out[0, h], out[0, (h // 4) * 4])


def test_decode_block_permutation_invariance_bitexact(dev):
    say("decode block permutation invariance")
    rng = np.random.default_rng(6)
    hkv, bs, d, hq, nb = 8, 16, 128, 32, 300
    ctx = np.int32([700, 1300, 33])
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d, "bf16")
    tables = make_tables(rng, ctx, bs, nb)
    q = rng.standard_normal((3, hq, d)).astype(np.float32)
    a = run_gpu(dev, q, kp, vp, tables, ctx, 0.08)
    perm = rng.permutation(nb).astype(np.int32)
    kp2, vp2 = np.empty_like(kp), np.empty_like(vp)
    kp2[perm], vp2[perm] = kp, vp
    tab2 = np.where(tables >= 0, perm[np.maximum(tables, 0)], -1).astype(np.int32)
    b = run_gpu(dev, q, kp2, vp2, tab2, ctx, 0.08)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_decode_invalid_blocks_and_context_clamp(dev, dtype):
    say(f"decode invalid block ids / clamp dtype={dtype}")
    rng = np.random.default_rng(7)
    hkv, bs, d, hq = 2, 16, 64, 4
    ctx = np.int32([300, 5000])  # 5000 > max_blocks*bs: clamped to 320
    q, kp, vp, _, _, tables = case(7, 2, hq, hkv, d, np.int32([320, 320]), dtype)
    tables[0, 4] = -1          # invalid ids: those tokens are left out
    tables[0, 7] = 10 ** 6
    scale = 0.125
    got = run_gpu(dev, q, kp, vp, tables, ctx, scale)
    want = oracle.decode_attention(q, kp, vp, tables, ctx, scale)
    assert_allclose_ref(got, want, RTOL, ATOL, "invalid blocks")
    # max_context below the real lengths clamps them too
    got = run_gpu(dev, q, kp, vp, tables, ctx, scale, max_context=100)
    want = oracle.decode_attention(q, kp, vp, tables[:, :7], np.minimum(ctx, 100).astype(np.int32),
                                   scale)
    assert_allclose_ref(got, want, RTOL, ATOL, "max_context clamp")


def test_decode_config2_full_shape(dev):
    """Config 2: B64, Hq32, Hkv8, D128, BS16, bf16, L ~ U[512, 4096]."""
    say("decode config-2 full shape")
    ctx = contexts(np.random.default_rng(2), 64, 512, 4096)
    (q, k, v, t, c), (qh, kh, vh, th, ch) = device_case(dev, 2, 64, 32, 8, 128, ctx)
    scale = float(np.float32(1.0 / math.sqrt(128)))
    got = to_np(kv.decode_attention(q, k, v, t, c, scale, max_context=4096))
    want = oracle.decode_attention(qh, kh, vh, th, ch, scale, n_threads=16)
    assert_allclose_ref(got, want, RTOL, ATOL, "config 2 vs oracle (bf16 pool)")
    # against fp32 K/V that the bf16 pool rounds (a subset of sequences: the
    # unrounded pool is regenerated from the same seed in fp32)
    (_, k32, v32, _, _), (_, kf, vf, _, _) = device_case(dev, 2, 64, 32, 8, 128, ctx,
                                                         dtype=torch.float32)
    sub = slice(0, 8)
    want32 = oracle.decode_attention(qh[sub], kf, vf, th[sub], ch[sub], scale, n_threads=16)
    assert np.abs(got[sub] - want32).max() <= BF16_VS_F32_ATOL


def test_decode_config3_long_context_splitk(dev):
    """Config 3: B8, Hq32, Hkv8, D128, bf16, L ~ U[16384, 65536], permuted
    non-contiguous blocks; many partitions per sequence through the merge."""
    say("decode config-3 long context")
    ctx = contexts(np.random.default_rng(3), 8, 16384, 65536)
    (q, k, v, t, c), (qh, kh, vh, th, ch) = device_case(dev, 3, 8, 32, 8, 128, ctx)
    scale = float(np.float32(1.0 / math.sqrt(128)))
    got = to_np(kv.decode_attention(q, k, v, t, c, scale, max_context=65536))
    want = oracle.decode_attention(qh, kh, vh, th, ch, scale, n_threads=16)
    assert_allclose_ref(got, want, RTOL, ATOL, "config 3 vs oracle (bf16 pool)")
    split, _ = oracle.decode_splitk(qh, kh, vh, th, ch, scale, 256)
    assert_allclose_ref(got, split, RTOL, ATOL, "config 3 vs oracle split-K")


def test_decode_two_passes_match_fused_call(dev):
    say("decode two launches vs one call")
    rng = np.random.default_rng(8)
    ctx = contexts(rng, 16, 100, 3000)
    q, kp, vp, _, _, tables = case(8, 16, 32, 8, 128, ctx, "bf16")
    args = [to_dev(x, dev) for x in (q, kp, vp, tables, ctx)]
    ws = torch.empty(kv.workspace_bytes(16, 32, 128, 3008), dtype=torch.uint8, device=dev)
    a = kv.decode_attention(*args, 0.1, max_context=3008)
    b = torch.empty_like(a)
    kv.decode_attention(*args, 0.1, max_context=3008, out=b, workspace=ws, passes="partitions")
    kv.decode_attention(*args, 0.1, max_context=3008, out=b, workspace=ws, passes="merge")
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("hq,hkv,d", [(8, 2, 128), (8, 8, 64), (16, 2, 32)])
def test_decode_many_sequences_with_empty_ones(dev, hq, hkv, d):
    """More than 64 sequences (the work plan scans lengths 64 at a time),
    empty sequences between long ones, lengths on tile boundaries."""
    say(f"decode many sequences hq={hq} hkv={hkv} d={d}")
    rng = np.random.default_rng(hq * 7 + d)
    ctx = rng.integers(0, 700, size=300).astype(np.int32)
    ctx[::7] = 0
    ctx[3::11] = 16 * rng.integers(1, 40, size=len(ctx[3::11]))
    ctx[5] = 1
    q, kp, vp, _, _, tables = case(9, len(ctx), hq, hkv, d, ctx, "bf16")
    scale = float(np.float32(1.0 / math.sqrt(d)))
    got = run_gpu(dev, q, kp, vp, tables, ctx, scale)
    want = oracle.decode_attention(q, kp, vp, tables, ctx, scale, n_threads=16)
    assert_allclose_ref(got, want, RTOL, ATOL, "many sequences vs oracle")
    assert not got[ctx == 0].any()


def test_decode_is_deterministic(dev):
    say("decode run-to-run determinism")
    rng = np.random.default_rng(10)
    ctx = contexts(rng, 40, 1, 5000)
    q, kp, vp, _, _, tables = case(10, 40, 32, 8, 128, ctx, "bf16")
    a = run_gpu(dev, q, kp, vp, tables, ctx, 0.09)
    b = run_gpu(dev, q, kp, vp, tables, ctx, 0.09)
    assert np.array_equal(a, b)


def test_decode_graph_replay_matches_eager(dev):
    """Decode calls of several layers (partition + merge passes) captured in
    one HIP graph, as the bench and a serving step replay them: every replay,
    with new queries written eagerly between replays, equals the eager calls
    bit for bit."""
    say("decode graph replay")
    rng = np.random.default_rng(12)
    ctx = contexts(rng, 24, 1, 3000)
    layers = []
    for i in range(3):
        q, kp, vp, _, _, tables = case(20 + i, 24, 32, 8, 128, ctx, "bf16")
        layers.append([to_dev(q, dev), to_dev(kp, dev), to_dev(vp, dev), to_dev(tables, dev)])
    ctx_d = to_dev(ctx, dev)
    mc = 3008
    ws = torch.zeros(kv.workspace_bytes(24, 32, 128, mc), dtype=torch.uint8, device=dev)
    outs = [torch.zeros_like(l[0]) for l in layers]

    def step(dst):
        for (q, k, v, t), o in zip(layers, dst):
            kv.decode_attention(q, k, v, t, ctx_d, 0.09, max_context=mc, out=o, workspace=ws)

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(outs)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(outs)
    g = torch.Generator(device=dev).manual_seed(3)
    for rep in range(4):
        for l in layers:
            l[0].normal_(generator=g)
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = [torch.zeros_like(o) for o in outs]
        step(eager)
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep}"


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("P", [64, 192, 320, 512, 576, 640])
def test_decode_caller_partition_sizes(dev, dtype, P):
    """Every accepted partition size (multiples of 64 tokens up to 640) gives
    the oracle's result: sizes up to 512 run on the 512-token build, larger
    ones on the 640-token build, with the slots past the size masked; the
    contexts straddle the partition and block boundaries."""
    ctx = np.array([1, 63, 64, 65, 511, 512, 513, 575, 577, 640, 641, 1300, 2048, 3333], np.int32)
    say(f"decode partition_size={P} dtype={dtype}")
    q, kp, vp, kf, vf, tables = case(P + 7, len(ctx), 32, 8, 128, ctx, dtype)
    scale = float(np.float32(1.0 / math.sqrt(128)))
    out = kv.decode_attention(to_dev(q, dev), to_dev(kp, dev), to_dev(vp, dev), to_dev(tables, dev),
                              to_dev(ctx, dev), scale, partition_size=P)
    torch.cuda.synchronize()
    want = oracle.decode_attention(q, kp, vp, tables, ctx, scale)
    assert_allclose_ref(to_np(out), want, RTOL, ATOL, f"partition {P} vs oracle")


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (16, 2, 128), (8, 8, 64), (8, 4, 32),
                                      (64, 8, 128)])
@pytest.mark.parametrize("P", [768, 896, 1024, 1280, 0])
def test_decode_wide_partitions_bf16(dev, P, hq, hkv, d):
    """bf16 pools: the 8-wave builds (768 and 1280 tokens; sizes between run
    on the 1280-token build with the slots past the size masked) and the
    default for the call's max_context give the oracle's result for every
    group size and head dim, with contexts straddling partition and block
    boundaries and a sequence long enough for many partitions."""
    ctx = np.array([1, 127, 128, 129, 767, 768, 769, 1279, 1280, 1281, 2047, 4100, 9000, 0],
                   np.int32)
    say(f"decode wide partition_size={P} hq={hq} hkv={hkv} d={d}")
    q, kp, vp, kf, vf, tables = case(P + hq + d, len(ctx), hq, hkv, d, ctx, "bf16")
    scale = float(np.float32(1.0 / math.sqrt(d)))
    out = kv.decode_attention(to_dev(q, dev), to_dev(kp, dev), to_dev(vp, dev), to_dev(tables, dev),
                              to_dev(ctx, dev), scale, partition_size=P)
    torch.cuda.synchronize()
    want = oracle.decode_attention(q, kp, vp, tables, ctx, scale)
    assert_allclose_ref(to_np(out), want, RTOL, ATOL, f"wide partition {P} vs oracle")


@pytest.mark.parametrize("max_context", [None, 1000])
@pytest.mark.parametrize("P", [0, 256, 640, 768, 1280])
@pytest.mark.parametrize("hq,hkv,d", [(4, 4, 32), (8, 4, 64), (32, 8, 128), (8, 1, 128),
                                      (16, 2, 128)])
def test_decode_append_fused_matches_append_then_decode(dev, max_context, P, hq, hkv, d):
    """rkv_decode_attention_append == rkv_append of the new rows followed by
    rkv_decode_attention, bit for bit in the pools and the output: new tokens
    at the first row of a block, mid-block and at the last row, at partition
    boundaries of every build, a sequence whose new block id is invalid (-1
    and past the pool: nothing written, the tile masked), an empty sequence,
    and (max_context 1000) sequences clamped below their length, whose rows
    are not written.  Every case is also checked against the oracle on the
    appended pool, over the lengths clamped to max_context."""
    bs = 16
    ctx = np.array([1, 2, 16, 17, 640, 641, 768, 769, 1280, 1281, 4100, 0, 40, 50, 33],
                   np.int32)
    say(f"decode append fused P={P} hq={hq} hkv={hkv} d={d} max_context={max_context}")
    q, kp, vp, kf, vf, tables = case(7 * P + hq + d, len(ctx), hq, hkv, d, ctx, "bf16")
    nb = kp.shape[0]
    tables[12, (40 - 1) // bs] = -1          # the new token's block: not a block
    tables[13, (50 - 1) // bs] = nb + 3      # past the pool
    rng = np.random.default_rng(P + d)
    kn = rng.standard_normal((len(ctx), hkv, d)).astype(np.float32)
    vn = rng.standard_normal((len(ctx), hkv, d)).astype(np.float32)
    cap = min(max_context if max_context is not None else 1 << 30, tables.shape[1] * bs)
    slots = np.full(len(ctx), -1, np.int64)
    for b, L in enumerate(ctx):
        if 0 < L <= cap:
            blk = int(tables[b, (L - 1) // bs])
            slots[b] = blk * bs + (L - 1) % bs if 0 <= blk < nb else -1
    scale = float(np.float32(1.0 / math.sqrt(d)))
    qd, td, cd = to_dev(q, dev), to_dev(tables, dev), to_dev(ctx, dev)
    knd, vnd = to_dev(kn, dev), to_dev(vn, dev)
    k1, v1 = to_dev(kp, dev), to_dev(vp, dev)
    k2, v2 = k1.clone(), v1.clone()
    kv.append(k1, v1, knd, vnd, to_dev(slots, dev))
    want = kv.decode_attention(qd, k1, v1, td, cd, scale, max_context=max_context,
                               partition_size=P)
    got = kv.decode_attention_append(qd, k2, v2, knd, vnd, td, cd, scale,
                                     max_context=max_context, partition_size=P)
    torch.cuda.synchronize()
    assert torch.equal(k2.view(torch.int16), k1.view(torch.int16)), "K pool differs"
    assert torch.equal(v2.view(torch.int16), v1.view(torch.int16)), "V pool differs"
    assert torch.equal(got, want), f"max diff {(got - want).abs().max().item()}"
    ref = oracle.decode_attention(q, to_np(k1), to_np(v1), tables, np.minimum(ctx, cap), scale)
    assert_allclose_ref(to_np(got), ref, RTOL, ATOL, "fused append vs oracle")
