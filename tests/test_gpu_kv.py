"""GPU parity of append / gather / copy_blocks against the oracle: bit-exact."""
import numpy as np
import pytest
import torch

import oracle
from rustral_amd import kv
from tests.gpu_util import say, to_dev, to_np
from tests.helpers import contexts, make_pool, make_tables

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("hkv,d", [(8, 128), (4, 32), (2, 64)])
def test_append_bitexact(dev, dtype, hkv, d):
    say(f"append dtype={dtype} hkv={hkv} d={d}")
    rng = np.random.default_rng(100 + d)
    nb, bs, n = 50, 16, 300
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d, dtype)
    slots = rng.permutation(nb * bs)[:n].astype(np.int64)
    slots[::37] = -1
    slots[5] = nb * bs + 1000  # out of range: skipped on both sides
    kn = rng.standard_normal((n, hkv, d)).astype(np.float32)
    vn = rng.standard_normal((n, hkv, d)).astype(np.float32)
    gk, gv = to_dev(kp, dev), to_dev(vp, dev)
    kv.append(gk, gv, to_dev(kn, dev), to_dev(vn, dev), to_dev(slots, dev))
    oracle.append(kp, vp, kn, vn, slots)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(gk), kp)
    assert np.array_equal(to_np(gv), vp)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_append_multi_layer_one_launch(dev, dtype):
    say(f"append multi-layer dtype={dtype}")
    rng = np.random.default_rng(7)
    nl, nb, hkv, bs, d, n = 4, 40, 8, 16, 128, 64
    kp = np.zeros((nl, nb, hkv, bs, d), np.float32)
    vp = np.zeros_like(kp)
    if dtype == "bf16":
        kp, vp = kp.astype(np.uint16), vp.astype(np.uint16)
    slots = rng.permutation(nb * bs)[:n].astype(np.int64)
    kn = rng.standard_normal((nl, n, hkv, d)).astype(np.float32)
    vn = rng.standard_normal((nl, n, hkv, d)).astype(np.float32)
    gk, gv = to_dev(kp, dev), to_dev(vp, dev)
    kv.append(gk, gv, to_dev(kn, dev), to_dev(vn, dev), to_dev(slots, dev))
    for l in range(nl):
        oracle.append(kp[l], vp[l], kn[l], vn[l], slots)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(gk), kp) and np.array_equal(to_np(gv), vp)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("hkv,d,bs", [(32, 128, 16), (8, 128, 12), (3, 40, 5)])
def test_append_wide_rows_and_other_block_sizes(dev, dtype, hkv, d, bs):
    """Hkv*D/8 above the 256-thread workgroup (the kernel's chunk loop) and
    block sizes that are not a power of two (slot / block_size by division)."""
    say(f"append wide/odd dtype={dtype} hkv={hkv} d={d} bs={bs}")
    rng = np.random.default_rng(hkv * 1000 + d + bs)
    n = 200
    nb = n // bs + 10
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d, dtype)
    slots = rng.permutation(nb * bs)[:n].astype(np.int64)
    slots[::11] = -1
    kn = rng.standard_normal((n, hkv, d)).astype(np.float32)
    vn = rng.standard_normal((n, hkv, d)).astype(np.float32)
    gk, gv = to_dev(kp, dev), to_dev(vp, dev)
    kv.append(gk, gv, to_dev(kn, dev), to_dev(vn, dev), to_dev(slots, dev))
    oracle.append(kp, vp, kn, vn, slots)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(gk), kp)
    assert np.array_equal(to_np(gv), vp)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_append_graph_replay_matches_eager(dev, dtype):
    """Per-step appends captured in a HIP graph (as a serving loop captures a
    step): every replay, with eager work and synchronisation between the
    replays, writes exactly what the eager calls write."""
    say(f"append graph replay dtype={dtype}")
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    nl, nb, hkv, bs, d, n = 3, 64, 8, 16, 128, 48
    g = torch.Generator(device=dev).manual_seed(5)
    perm = torch.randperm(nb * bs, generator=g, device=dev)
    slot_sets = [perm[i * n:(i + 1) * n].to(torch.int64).contiguous() for i in range(4)]
    kn = torch.empty((nl, n, hkv, d), device=dev)
    vn = torch.empty_like(kn)
    kp = torch.zeros((nl, nb, hkv, bs, d), dtype=tdt, device=dev)
    vp = torch.zeros_like(kp)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):                      # warm-up outside the capture
        for s in slot_sets:
            kv.append(kp, vp, kn.normal_(generator=g), vn.normal_(generator=g), s)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for s in slot_sets:
            kv.append(kp, vp, kn, vn, s)
    for rep in range(4):
        kp.zero_(), vp.zero_()
        kn.normal_(generator=g), vn.normal_(generator=g)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ek, ev = torch.zeros_like(kp), torch.zeros_like(vp)
        for s in slot_sets:
            kv.append(ek, ev, kn, vn, s)
        torch.cuda.synchronize()
        assert torch.equal(kp, ek) and torch.equal(vp, ev), f"replay {rep}"
        assert int((kp != 0).sum()) > 0


@pytest.mark.parametrize("out_f32", [False, True])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_gather_bitexact_padded_and_packed(dev, dtype, out_f32):
    say(f"gather dtype={dtype} out_f32={out_f32}")
    rng = np.random.default_rng(11)
    nb, hkv, bs, d = 400, 8, 16, 128
    ctx = np.array([0, 1, 15, 16, 17, 255, 1000, 2049], np.int32)
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d, dtype)
    tables = make_tables(rng, ctx, bs, nb)
    tables[6, 3] = nb + 7  # invalid block id: its rows stay untouched
    gk, gv = to_dev(kp, dev), to_dev(vp, dev)
    gt, gc = to_dev(tables, dev), to_dev(ctx, dev)
    odt = torch.float32 if out_f32 else None
    ko, vo = kv.gather(gk, gv, gt, gc, max_ctx=int(ctx.max()), out_dtype=odt)
    rk, rv = oracle.gather(kp, vp, tables, ctx, max_ctx=int(ctx.max()), out_f32=out_f32)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(ko), rk) and np.array_equal(to_np(vo), rv)
    sizes = ctx.astype(np.int64) * hkv * d
    off = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    total = int(sizes.sum())
    ko, vo = kv.gather(gk, gv, gt, gc, out_offsets=to_dev(off, dev), out_total=total,
                       out_dtype=odt)
    rk, rv = oracle.gather(kp, vp, tables, ctx, out_offsets=off, out_f32=out_f32)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(ko), rk) and np.array_equal(to_np(vo), rv)


@pytest.mark.parametrize("out_f32", [False, True])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("hkv,bs,d", [(1, 16, 32), (2, 12, 64), (3, 8, 40), (8, 32, 96),
                                      (4, 16, 128), (8, 24, 128)])
def test_gather_block_sizes_head_dims_and_guards(dev, dtype, out_f32, hkv, bs, d):
    """Block sizes that are and are not powers of two, head dims with and
    without a specialised build, blocks that fill whole rounds of the
    kernel and blocks that do not, partial last blocks: the packed output
    equals the oracle's, and guard rows after every sequence stay
    untouched."""
    say(f"gather hkv={hkv} bs={bs} d={d} dtype={dtype} out_f32={out_f32}")
    rng = np.random.default_rng(hkv * 100 + bs + d)
    nb = 64
    ctx = np.array([bs * 3, 1, bs - 1, 0, bs * 7 + 5, bs + 1], np.int32)
    kp, vp, _, _ = make_pool(rng, nb, hkv, bs, d, dtype)
    tables = make_tables(rng, ctx, bs, nb)
    gap = hkv * d
    sizes = ctx.astype(np.int64) * hkv * d + gap
    off = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    total = int(sizes.sum())
    odt = torch.float32 if (out_f32 or dtype == "f32") else torch.bfloat16
    guard = -3.5
    ko = torch.full((total,), guard, dtype=odt, device=dev)
    vo = torch.full((total,), guard, dtype=odt, device=dev)
    kv.gather(to_dev(kp, dev), to_dev(vp, dev), to_dev(tables, dev), to_dev(ctx, dev),
              out_offsets=to_dev(off, dev), out_total=total, out_dtype=odt, k_out=ko, v_out=vo)
    torch.cuda.synchronize()
    np_dt = np.float32 if odt == torch.float32 else np.uint16
    g = np.float32(guard) if np_dt == np.float32 else oracle.bf16_from_f32(np.float32([guard]))[0]
    rk = np.full(total, g, np_dt)
    rv = np.full(total, g, np_dt)
    oracle.gather(kp, vp, tables, ctx, out_offsets=off, out_f32=out_f32, k_out=rk, v_out=rv)
    assert np.array_equal(to_np(ko), rk) and np.array_equal(to_np(vo), rv)
    for b in range(len(ctx)):
        g0 = int(off[b] + ctx[b] * hkv * d)
        assert (rk[g0:g0 + gap] == g).all()


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_gather_of_append_roundtrip_config1_shape(dev, dtype):
    """Config-1 shape (Hkv 8, D 128, BS 16, 65,536-block pool, 64 sequences with
    contexts U[512, 4096]), two layers, both storage types (the fp32 pool is
    4 GiB per layer for K and for V): append every token of every sequence,
    gather, and get the appended rows back bit for bit (bf16 pool: their RNE
    rounding, checked against the oracle's bit routine)."""
    say(f"append+gather round trip, config-1 shape, {dtype}")
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    bits = torch.int16 if dtype == "bf16" else torch.int32
    rng = np.random.default_rng(1)
    nl, nb, hkv, bs, d, B = 2, 65536, 8, 16, 128, 64
    ctx = contexts(rng, B, 512, 4096)
    tables = make_tables(rng, ctx, bs, nb, max_blocks=4096 // bs)
    pos = [np.arange(L) for L in ctx]
    slots = np.concatenate([tables[b, p // bs].astype(np.int64) * bs + p % bs
                            for b, p in enumerate(pos)])
    n = slots.shape[0]
    g = torch.Generator(device=dev).manual_seed(1)
    kn = torch.randn((nl, n, hkv, d), generator=g, device=dev)
    vn = torch.randn((nl, n, hkv, d), generator=g, device=dev)
    gk = torch.zeros((nl, nb, hkv, bs, d), dtype=tdt, device=dev)
    gv = torch.zeros_like(gk)
    kv.append(gk, gv, kn, vn, to_dev(slots, dev))
    gt, gc = to_dev(tables, dev), to_dev(ctx, dev)
    offs = np.concatenate([[0], np.cumsum(ctx.astype(np.int64))[:-1]])
    for l in range(nl):
        ko, vo = kv.gather(gk[l], gv[l], gt, gc, max_ctx=4096)
        # compare a strided subset of sequences on the host, all of them on device
        for b in range(0, B, 9):
            L = int(ctx[b])
            src = kn[l, offs[b]:offs[b] + L].cpu().numpy()
            want_k = (oracle.bf16_from_f32(src) if dtype == "bf16" else src).transpose(1, 0, 2)
            assert np.array_equal(to_np(ko[b, :, :L]), want_k)
        for b in range(B):
            L = int(ctx[b])
            sk = kn[l, offs[b]:offs[b] + L].to(tdt).transpose(0, 1)
            sv = vn[l, offs[b]:offs[b] + L].to(tdt).transpose(0, 1)
            assert torch.equal(ko[b, :, :L].view(bits), sk.contiguous().view(bits))
            assert torch.equal(vo[b, :, :L].view(bits), sv.contiguous().view(bits))
        del ko, vo
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_copy_blocks_bitexact_multi_layer(dev, dtype):
    say(f"copy_blocks dtype={dtype}")
    rng = np.random.default_rng(13)
    nl, nb, hkv, bs, d = 3, 200, 8, 16, 128
    kp = rng.standard_normal((nl, nb, hkv, bs, d)).astype(np.float32)
    vp = rng.standard_normal((nl, nb, hkv, bs, d)).astype(np.float32)
    if dtype == "bf16":
        kp, vp = oracle.bf16_from_f32(kp), oracle.bf16_from_f32(vp)
    perm = rng.permutation(nb)
    pairs = np.stack([perm[:60], perm[60:120]], axis=1).astype(np.int32)
    pairs = np.concatenate([pairs, [[1, nb], [-5, 3]]]).astype(np.int32)
    gk, gv = to_dev(kp, dev), to_dev(vp, dev)
    kv.copy_blocks(gk, gv, to_dev(pairs, dev))
    oracle.copy_blocks(kp, vp, pairs)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(gk), kp) and np.array_equal(to_np(gv), vp)


def test_empty_calls_are_no_ops(dev):
    say("empty calls")
    gk = torch.zeros((4, 2, 16, 32), device=dev)
    gv = torch.zeros_like(gk)
    kv.append(gk, gv, torch.zeros((0, 2, 32), device=dev), torch.zeros((0, 2, 32), device=dev),
              torch.zeros((0,), dtype=torch.int64, device=dev))
    kv.copy_blocks(gk, gv, torch.zeros((0, 2), dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    assert not gk.any()
