"""ctypes binding of librkv_ceiling.so: stream kernels that measure what HBM
delivers on this part for the access patterns of the paged-KV kernels (flat
read / write / copy, block copies, the decode kernel's tile loads with the
arithmetic removed).  A measurement aid for ``bench.py --workload
ceilings``, not part of the product ABI; torch supplies the device buffers
and the stream."""
from __future__ import annotations

import ctypes as C
import os

from rustral_amd.build import LIB_DIR

CEILING_LIB = os.path.join(LIB_DIR, "librkv_ceiling.so")

_SIG = {
    "rkvc_read": [C.c_void_p, C.c_int64, C.c_void_p, C.c_uint, C.c_int, C.c_void_p],
    "rkvc_write": [C.c_void_p, C.c_int64, C.c_int, C.c_void_p],
    "rkvc_copy": [C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_void_p],
    "rkvc_write_var": [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p],
    "rkvc_copy_var": [C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p],
    "rkvc_block_copy_pipe": [C.c_void_p, C.c_void_p, C.c_int, C.c_int64, C.c_int, C.c_void_p],
    "rkvc_read_unr": [C.c_void_p, C.c_int64, C.c_void_p, C.c_uint, C.c_int, C.c_int, C.c_void_p],
    "rkvc_write_unr": [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p],
    "rkvc_copy_unr": [C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_int, C.c_void_p],
    "rkvc_block_copy_unr": [C.c_void_p, C.c_void_p, C.c_int, C.c_int64, C.c_int64, C.c_int,
                            C.c_void_p],
    "rkvc_block_copy": [C.c_void_p, C.c_void_p, C.c_int, C.c_int64, C.c_int64, C.c_void_p],
    "rkvc_tile_stream": [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                         C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int64, C.c_int, C.c_void_p,
                         C.c_uint, C.c_void_p],
    "rkvc_tile_stream_shape": [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int,
                               C.c_int, C.c_int64, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_uint,
                               C.c_void_p],
    "rkvc_nth": [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_int, C.c_int64,
                 C.c_int64, C.c_int, C.c_void_p],
    "rkvc_tile_stream_1b": [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                            C.c_void_p, C.c_int, C.c_int, C.c_int64, C.c_int, C.c_int,
                            C.c_void_p, C.c_uint, C.c_void_p],
}
_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        # torch first: its HIP runtime (soname libamdhip64.so.7) is then the
        # one this library binds to, so torch's buffers and streams are valid
        # here; loaded the other way round the process holds two runtimes
        import torch  # noqa: F401
        if not os.path.exists(CEILING_LIB):
            raise ImportError(f"{CEILING_LIB} is missing: build it with `python -m rustral_amd.build`")
        L = C.CDLL(CEILING_LIB)
        for name, args in _SIG.items():
            fn = getattr(L, name)
            fn.restype = C.c_int
            fn.argtypes = args
        _lib = L
    return _lib


def _stream(torch, dev):
    return C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _ok(rc: int, what: str) -> None:
    if rc < 0:
        raise ValueError(f"{what}: invalid argument")
    if rc > 0:
        raise RuntimeError(f"{what}: launch failed (hipError_t {rc})")


def read(torch, buf, sink, grid: int = 4096) -> None:
    _ok(lib().rkvc_read(buf.data_ptr(), buf.numel() * buf.element_size(), sink.data_ptr(),
                        0x9E3779B9, grid, _stream(torch, buf.device)), "rkvc_read")


def write(torch, buf, grid: int = 8192) -> None:
    _ok(lib().rkvc_write(buf.data_ptr(), buf.numel() * buf.element_size(), grid,
                         _stream(torch, buf.device)), "rkvc_write")


def copy(torch, src, dst, grid: int = 8192) -> None:
    n = src.numel() * src.element_size()
    assert dst.numel() * dst.element_size() >= n
    _ok(lib().rkvc_copy(src.data_ptr(), dst.data_ptr(), n, grid, _stream(torch, src.device)),
        "rkvc_copy")


WRITE_NT, TWO_PER_LANE, CHUNKED, LOAD_NT = 1, 2, 4, 8


def write_var(torch, buf, grid: int, variant: int) -> None:
    """Flat write of buf with the variant bits WRITE_NT | TWO_PER_LANE | CHUNKED."""
    _ok(lib().rkvc_write_var(buf.data_ptr(), buf.numel() * buf.element_size(), grid, variant,
                             _stream(torch, buf.device)), "rkvc_write_var")


def copy_var(torch, src, dst, grid: int, variant: int) -> None:
    """Flat copy with the variant bits of write_var plus LOAD_NT."""
    n = src.numel() * src.element_size()
    assert dst.numel() * dst.element_size() >= n
    _ok(lib().rkvc_copy_var(src.data_ptr(), dst.data_ptr(), n, grid, variant,
                            _stream(torch, src.device)), "rkvc_copy_var")


def block_copy(torch, pool, pairs, block_bytes: int) -> None:
    """pairs: int32 [n, 2] (src, dst) on the device; pool: the blocks."""
    nb = pool.numel() * pool.element_size() // block_bytes
    _ok(lib().rkvc_block_copy(pool.data_ptr(), pairs.data_ptr(), pairs.shape[0], block_bytes, nb,
                              _stream(torch, pool.device)), "rkvc_block_copy")


def read_unr(torch, buf, sink, unr: int, grid: int = 0) -> None:
    """Flat nontemporal read, unr 16-byte units a thread per round (grid 0:
    one round per workgroup)."""
    _ok(lib().rkvc_read_unr(buf.data_ptr(), buf.numel() * buf.element_size(), sink.data_ptr(),
                            0x9E3779B9, unr, grid, _stream(torch, buf.device)), "rkvc_read_unr")


def write_unr(torch, buf, unr: int, grid: int = 0) -> None:
    """Flat write, unr 16-byte units a thread per round (grid 0: one round
    per workgroup)."""
    _ok(lib().rkvc_write_unr(buf.data_ptr(), buf.numel() * buf.element_size(), unr, grid,
                             _stream(torch, buf.device)), "rkvc_write_unr")


def copy_unr(torch, src, dst, unr: int, grid: int = 0, nt: bool = True) -> None:
    n = src.numel() * src.element_size()
    assert dst.numel() * dst.element_size() >= n
    _ok(lib().rkvc_copy_unr(src.data_ptr(), dst.data_ptr(), n, unr, grid, int(nt),
                            _stream(torch, src.device)), "rkvc_copy_unr")


def block_copy_unr(torch, pool, pairs, block_bytes: int, unr: int) -> None:
    """Block copies split into (unr * 4 KiB)-byte pieces, one workgroup each."""
    nb = pool.numel() * pool.element_size() // block_bytes
    _ok(lib().rkvc_block_copy_unr(pool.data_ptr(), pairs.data_ptr(), pairs.shape[0], block_bytes,
                                  nb, unr, _stream(torch, pool.device)), "rkvc_block_copy_unr")


def block_copy_pipe(torch, pool, pairs, grid: int) -> None:
    """32 KiB block copies, each workgroup a grid-stride run of pairs with the
    next pair's loads issued before the current pair's stores."""
    nb = pool.numel() * pool.element_size() // 32768
    _ok(lib().rkvc_block_copy_pipe(pool.data_ptr(), pairs.data_ptr(), pairs.shape[0], nb, grid,
                                   _stream(torch, pool.device)), "rkvc_block_copy_pipe")


def tile_stream(torch, k_pool, v_pool, tables, ctx_lens, sink, partitions: int,
                k_scale=None, v_scale=None) -> None:
    """Pools [num_blocks, Hkv, 16, 128] of bf16, or of 1-byte elements with
    fp32 scales [num_blocks, Hkv, 16]; tables int32 [B, max_blocks]."""
    nb, hkv = k_pool.shape[0], k_pool.shape[1]
    eb = k_pool.element_size()
    ks = k_scale.data_ptr() if k_scale is not None else None
    vs = v_scale.data_ptr() if v_scale is not None else None
    _ok(lib().rkvc_tile_stream(k_pool.data_ptr(), v_pool.data_ptr(), ks, vs, eb,
                               tables.data_ptr(), tables.shape[1], ctx_lens.data_ptr(),
                               tables.shape[0], hkv, nb, partitions, sink.data_ptr(), 0x9E3779B9,
                               _stream(torch, k_pool.device)), "rkvc_tile_stream")


TILE_STREAM_1B = {"row_scales": 0, "no_scales": 1, "two_heads_per_wave": 2,
                  "four_heads_per_wave": 3, "partition_major": 4, "scales_after_k_tile": 5}


def tile_stream_1b(torch, k_pool, v_pool, tables, ctx_lens, sink, partitions: int,
                   variant: str, num_blocks: int, num_kv_heads: int,
                   k_scale=None, v_scale=None) -> None:
    """Variants of the 1-byte decode load pattern (D 128, 16-token blocks):
    k_pool / v_pool byte pools of num_blocks x num_kv_heads tiles (2,048
    bytes; the K pool's tiles 2,176 bytes for "scales_after_k_tile"),
    k_scale / v_scale fp32 [num_blocks, Hkv, 16] for the variants that read
    row scales."""
    ks = k_scale.data_ptr() if k_scale is not None else None
    vs = v_scale.data_ptr() if v_scale is not None else None
    _ok(lib().rkvc_tile_stream_1b(k_pool.data_ptr(), v_pool.data_ptr(), ks, vs,
                                  tables.data_ptr(), tables.shape[1], ctx_lens.data_ptr(),
                                  tables.shape[0], num_kv_heads, num_blocks, partitions,
                                  TILE_STREAM_1B[variant], sink.data_ptr(), 0x9E3779B9,
                                  _stream(torch, k_pool.device)), "rkvc_tile_stream_1b")


def write_nth(torch, buf, nth: int) -> None:
    """Flat write of buf, one 16-byte unit a thread, nth threads a workgroup."""
    _ok(lib().rkvc_nth(0, None, buf.data_ptr(), buf.numel() * buf.element_size(), None, 0, 0, 0,
                       nth, _stream(torch, buf.device)), "rkvc_nth write")


def copy_nth(torch, src, dst, nth: int) -> None:
    """Flat copy src -> dst (nontemporal), one unit a thread, nth threads a workgroup."""
    _ok(lib().rkvc_nth(1, src.data_ptr(), dst.data_ptr(), src.numel() * src.element_size(), None,
                       0, 0, 0, nth, _stream(torch, src.device)), "rkvc_nth copy")


def block_copy_nth(torch, pool, pairs, block_bytes: int, nth: int) -> None:
    """Block copies inside pool (pairs int32 [n, 2]), pieces of 16 nth bytes."""
    nb = pool.numel() * pool.element_size() // block_bytes
    _ok(lib().rkvc_nth(2, None, pool.data_ptr(), 0, pairs.data_ptr(), pairs.shape[0], block_bytes,
                       nb, nth, _stream(torch, pool.device)), "rkvc_nth block copy")


def tile_stream_shape(torch, k_pool, v_pool, tables, ctx_lens, sink, partitions: int,
                      tiles_per_wave: int, waves: int) -> None:
    """The bf16 decode pattern at (tiles a wave, waves a workgroup) = (10, 4),
    (6, 8) or (10, 8): the 640-, 768- and 1280-token partition builds."""
    nb, hkv = k_pool.shape[0], k_pool.shape[1]
    _ok(lib().rkvc_tile_stream_shape(k_pool.data_ptr(), v_pool.data_ptr(), tables.data_ptr(),
                                     tables.shape[1], ctx_lens.data_ptr(), tables.shape[0], hkv,
                                     nb, partitions, tiles_per_wave, waves, sink.data_ptr(),
                                     0x9E3779B9, _stream(torch, k_pool.device)),
        "rkvc_tile_stream_shape")
