"""ctypes binding of librustral_kv.so (the C ABI declared in include/rustral_kv.h).

The library is the only compute path: if it has not been built, importing
this module raises instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes as C
import os

from .build import LIB_PATH

RKV_F32, RKV_BF16 = 0, 1
RKV_OK = 0
RKV_ERR_INVALID_ARG, RKV_ERR_UNSUPPORTED, RKV_ERR_WORKSPACE, RKV_ERR_HIP = -1, -2, -3, -4

# Every symbol include/rustral_kv.h declares, with (restype, argtypes).
_p, _i, _i64, _f, _sz = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_size_t
SIGNATURES = {
    "rkv_last_error": (C.c_char_p, []),
    "rkv_version": (_i, []),
    "rkv_append": (_i, [_p, _p, _i64, _p, _p, _i64, _i64, _i64, _p, _i64, _i, _i, _i, _i, _i64,
                        _i, _p]),
    "rkv_gather": (_i, [_p, _p, _p, _p, _p, _i, _p, _p, _i, _i, _i, _i, _i64, _i, _i, _i, _p]),
    "rkv_copy_blocks": (_i, [_p, _p, _i64, _i, _p, _i, _i64, _i64, _p]),
    "rkv_decode_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "rkv_decode_partition_size": (_i, [_i, _i, _i]),
    "rkv_decode_attention": (_i, [_p, _p, _p, _p, _p, _i, _p, _i, _i, _i, _i, _i, _i64, _i, _f,
                                  _i, _i, _p, _sz, _p]),
    "rkv_decode_attention_partitions": (_i, [_p, _p, _p, _p, _p, _i, _p, _i, _i, _i, _i, _i,
                                             _i64, _i, _f, _i, _i, _p, _sz, _p]),
    "rkv_decode_attention_merge": (_i, [_p, _p, _i, _i, _i, _i, _i, _i, _i, _i, _p, _sz, _p]),
}


class RkvError(RuntimeError):
    """A non-zero status from the C ABI, with rkv_last_error()'s message."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[rkv {code}] {msg}")
        self.code = code


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m rustral_amd.build` "
                "(there is no fallback compute path)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != RKV_OK:
        raise RkvError(rc, lib().rkv_last_error().decode())
