"""The measurement library of ``bench.py --workload ceilings``
(rustral_amd/ceiling, librkv_ceiling.so): it loads and exports its stream
kernels (CPU); on the GPU its copies copy (bit-exact) and its read and
decode-pattern streams leave the sink untouched (their fold is stored
only when it equals a runtime value that no fold of these inputs takes)."""
import numpy as np
import pytest
import torch

from rustral_amd import ceiling as C

NAMES = ("rkvc_read", "rkvc_write", "rkvc_copy", "rkvc_block_copy", "rkvc_tile_stream",
         "rkvc_tile_stream_1b", "rkvc_nth", "rkvc_tile_stream_shape")


def test_library_loads_and_exports_the_stream_kernels():
    L = C.lib()
    for n in NAMES:
        assert hasattr(L, n), n


def test_arguments_are_checked_before_any_launch():
    L = C.lib()
    assert L.rkvc_read(None, 1 << 20, None, 0, 16, None) != 0
    assert L.rkvc_copy(None, None, 100, 16, None) != 0        # also not a multiple of 16
    assert L.rkvc_block_copy(None, None, 0, 32768, 1, None) != 0
    assert L.rkvc_tile_stream(None, None, None, None, 2, None, 0, None, 0, 0, 0, 0, None, 0,
                              None) != 0
    # the by-size kernels: a thread count outside 64..512, an unknown kind,
    # a size that is no multiple of 16, a block that is no whole number of
    # pieces
    assert L.rkvc_nth(0, None, None, 1 << 20, None, 0, 0, 0, 64, None) != 0
    assert L.rkvc_nth(3, None, None, 1 << 20, None, 0, 0, 0, 64, None) != 0
    assert L.rkvc_nth(0, None, 16, 1 << 20, None, 0, 0, 0, 96, None) != 0
    assert L.rkvc_nth(1, 16, 16, 100, None, 0, 0, 0, 64, None) != 0
    assert L.rkvc_nth(2, None, 16, 0, 16, 1, 1000, 4, 64, None) != 0
    # a partition shape the decode kernel has no build for
    assert L.rkvc_tile_stream_shape(16, 16, 16, 4, 16, 1, 8, 64, 1, 7, 8, 16, 0, None) != 0
    # the 1-byte pattern variants: an unknown variant, heads not divisible by
    # the heads per wave, scales missing where the variant reads them
    assert L.rkvc_tile_stream_1b(16, 16, 16, 16, 16, 4, 16, 1, 8, 64, 1, 6, 16, 0, None) != 0
    assert L.rkvc_tile_stream_1b(16, 16, 16, 16, 16, 4, 16, 1, 6, 64, 1, 3, 16, 0, None) != 0
    assert L.rkvc_tile_stream_1b(16, 16, None, None, 16, 4, 16, 1, 8, 64, 1, 0, 16, 0, None) != 0


@pytest.mark.gpu
def test_copies_are_bit_exact_and_streams_leave_the_sink(dev):
    from tests.gpu_util import say
    say("ceiling kernels: copy, block copy, read, tile stream")
    g = torch.Generator(device=dev).manual_seed(3)
    a = torch.randint(-2 ** 31, 2 ** 31 - 1, (1 << 22,), generator=g, dtype=torch.int32, device=dev)
    b = torch.zeros_like(a)
    C.copy(torch, a, b, grid=64)
    sink = torch.zeros(16, dtype=torch.int32, device=dev)
    C.read(torch, a, sink, grid=64)
    C.write(torch, b[: 1 << 20], grid=16)                     # rows 0 .. 2^20 rewritten
    torch.cuda.synchronize()
    assert torch.equal(a[1 << 20:], b[1 << 20:])
    assert int(sink.abs().sum()) == 0
    # block copy: 8 KiB blocks of a 16 MiB pool, disjoint sources and targets
    pool = a.clone()
    nblk, blk = pool.numel() * 4 // 8192, 8192
    rng = np.random.default_rng(1)
    perm = rng.permutation(nblk).astype(np.int32)
    pairs = np.stack([perm[:64], perm[64:128]], 1)
    C.block_copy(torch, pool, torch.from_numpy(pairs).to(dev), blk)
    torch.cuda.synchronize()
    want = a.cpu().numpy().reshape(nblk, -1).copy()
    want[pairs[:, 1]] = want[pairs[:, 0]]
    assert np.array_equal(pool.cpu().numpy().reshape(nblk, -1), want)
    # the decode pattern over a small bf16 pool (ids outside the pool are absent)
    nb, hkv = 64, 2
    k = torch.randn((nb, hkv, 16, 128), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn_like(k)
    tab = torch.tensor([[3, 9, -1, 70], [5, 6, 7, 8]], dtype=torch.int32, device=dev)
    ctx = torch.tensor([40, 64], dtype=torch.int32, device=dev)
    C.tile_stream(torch, k, v, tab, ctx, sink, partitions=1)
    for tpw, waves in ((10, 4), (6, 8), (10, 8)):
        C.tile_stream_shape(torch, k, v, tab, ctx, sink, 1, tpw, waves)
    k8 = torch.randint(0, 255, (nb, hkv, 16, 128), generator=g, dtype=torch.uint8, device=dev)
    v8 = torch.randint(0, 255, (nb, hkv, 16, 128), generator=g, dtype=torch.uint8, device=dev)
    ks = torch.rand((nb, hkv, 16), generator=g, device=dev)
    C.tile_stream(torch, k8, v8, tab, ctx, sink, partitions=1, k_scale=ks, v_scale=ks.clone())
    # the 1-byte pattern variants (the K pool of 2,176-byte tiles for the
    # scales-after-tile layout)
    kc = torch.randint(0, 255, (nb, hkv, 16 * 128 + 128), generator=g, dtype=torch.uint8,
                       device=dev)
    for variant in C.TILE_STREAM_1B:
        if variant == "four_heads_per_wave":   # needs a multiple of 4 KV heads (2 here)
            continue
        C.tile_stream_1b(torch, kc if variant == "scales_after_k_tile" else k8, v8, tab, ctx, sink,
                         1, variant, nb, hkv, k_scale=ks, v_scale=ks.clone())
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0
    # the by-size stream kernels copy bit-exactly at every workgroup size
    for nth in (64, 128, 256, 512):
        src = torch.randint(-2 ** 31, 2 ** 31 - 1, (1 << 20,), generator=g, dtype=torch.int32,
                            device=dev)
        dst = torch.zeros_like(src)
        C.copy_nth(torch, src, dst, nth)
        pool2 = a.clone()
        C.block_copy_nth(torch, pool2, torch.from_numpy(pairs).to(dev), blk, nth)
        C.write_nth(torch, dst[: 1 << 18], nth)         # the first 1 MiB rewritten
        torch.cuda.synchronize()
        assert torch.equal(src[1 << 18:], dst[1 << 18:]), nth
        assert np.array_equal(pool2.cpu().numpy().reshape(nblk, -1), want), nth
