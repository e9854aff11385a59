"""ctypes binding of librustral_kv.so (the C ABI declared in include/rustral_kv.h).

The library is the only compute path: if it has not been built, importing
this module raises instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes as C
import os

from .build import LIB_PATH

RKV_F32, RKV_BF16, RKV_I8, RKV_FP8 = 0, 1, 2, 3
RKV_OK = 0
RKV_ERR_INVALID_ARG, RKV_ERR_UNSUPPORTED, RKV_ERR_WORKSPACE, RKV_ERR_HIP = -1, -2, -3, -4
RKV_ERR_OOM = -5

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
    "rkv_decode_partition_size": (_i, [_i, _i, _i, _i]),
    "rkv_decode_partition_size_for": (_i, [_i, _i, _i, _i, _i, _i, _i]),
    "rkv_decode_attention": (_i, [_p, _p, _p, _p, _p, _i, _p, _i, _i, _i, _i, _i, _i64, _i, _f,
                                  _i, _i, _p, _sz, _p]),
    "rkv_decode_attention_append": (_i, [_p, _p, _p, _p, _p, _p, _p, _i, _p, _i, _i, _i, _i, _i,
                                         _i64, _i, _f, _i, _i, _p, _sz, _p]),
    "rkv_decode_attention_noalloc": (_i, [_p, _p, _p, _p, _p, _i, _p, _i, _i, _i, _i, _i, _i64,
                                          _i, _f, _i, _i, _p]),
    "rkv_decode_noalloc_max_bytes": (_sz, []),
    "rkv_decode_attention_partitions": (_i, [_p, _p, _p, _p, _p, _i, _p, _i, _i, _i, _i, _i,
                                             _i64, _i, _f, _i, _i, _p, _sz, _p]),
    "rkv_decode_attention_merge": (_i, [_p, _p, _i, _i, _i, _i, _i, _i, _i, _i, _p, _sz, _p]),
    "rkv_prefill_attention": (_i, [_p, _p, _p, _p, _p, _i, _p, _p, _i, _i, _i, _i, _i, _i64, _i,
                                   _f, _i, _p]),
    "rkv_append_q": (_i, [_p, _p, _p, _p, _i64, _p, _p, _i64, _i64, _i64, _p, _i64, _i, _i, _i,
                          _i, _i64, _i, _p]),
    "rkv_gather_q": (_i, [_p, _p, _p, _p, _p, _p, _p, _i, _p, _p, _i, _i, _i, _i, _i64, _i, _i,
                          _p]),
    "rkv_decode_attention_q": (_i, [_p, _p, _p, _p, _p, _p, _p, _i, _p, _i, _i, _i, _i, _i, _i64,
                                    _i, _f, _i, _i, _p, _sz, _p]),
    "rkv_decode_attention_append_q": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _p, _i, _i,
                                           _i, _i, _i, _i64, _i, _f, _i, _i, _p, _sz, _p]),
    # include/rustral_serving.h (host memory)
    "rkv_dbm_create": (_p, [_i64, _i, _i, _i, _p]),
    "rkv_dbm_destroy": (None, [_p]),
    "rkv_dbm_reserve": (_i, [_p, _p, _p, _i, _p]),
    "rkv_dbm_free": (_i, [_p, _p, _i, _p]),
    "rkv_dbm_slot_mapping": (_i, [_p, _p, _p, _i, _p, _p]),
    "rkv_dbm_batch_tables": (_i, [_p, _p, _i, _p, _i, _p]),
    "rkv_dbm_status": (_i, [_p, _p, _p, _i, _p]),
    "rkv_dbm_download": (_i, [_p, _p, _p, _p, _p, _p]),
    "rkv_bm_create": (_p, [_i64, _i]),
    "rkv_bm_destroy": (None, [_p]),
    "rkv_bm_allocate": (_i64, [_p, _i64, _i64, _p, _i64]),
    "rkv_bm_reserve": (_i64, [_p, _i64, _i64]),
    "rkv_bm_free": (_i64, [_p, _i64]),
    "rkv_bm_num_free": (_i64, [_p]),
    "rkv_bm_num_blocks": (_i64, [_p]),
    "rkv_bm_block_size": (_i, [_p]),
    "rkv_bm_table": (_i64, [_p, _i64, _p, _i64]),
    "rkv_bm_free_list": (_i64, [_p, _p, _i64]),
    "rkv_bm_fill_tables": (_i, [_p, _p, _i, _p, _i]),
    "rkv_bm_plan_compaction": (_i64, [_p, _i64, _p, _i64]),
    "rkv_bm_plan_migration": (_i64, [_p, _i64, _p, _i64]),
    "rkv_bm_plan_relocation": (_i64, [_p, _i64, _p, _i64]),
    "rkv_sched_create": (_p, [_i64, _i, _i, _i]),
    "rkv_sched_destroy": (None, [_p]),
    "rkv_sched_add_request": (_i64, [_p, _p, _i, _i, _i]),
    "rkv_sched_schedule": (_i, [_p]),
    "rkv_sched_batch_dims": (_i, [_p, _p, _p, _p]),
    "rkv_sched_batch": (_i, [_p, _p, _p, _p, _p, _p, _p, _i]),
    "rkv_sched_update": (_i, [_p, _p, _p, _i]),
    "rkv_sched_stats": (_i, [_p, _p]),
    "rkv_sched_generated": (_i64, [_p, _i64, _p, _i64]),
    "rkv_sched_block_manager": (_p, [_p]),
    "rkv_sampler_greedy": (_i, [_p, _i]),
    # include/rustral_model.h
    "rkv_embed": (_i, [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p]),
    "rkv_linear": (_i, [_p, _p, _p, _p, _i, _i, _i, _p]),
    "rkv_layer_norm": (_i, [_p, _p, _p, _p, _i, _i, _f, _p]),
    "rkv_qkv_append": (_i, [_p, _p, _p, _p, _p, _p, _p, _f, _p, _p, _p, _p, _p, _p, _i, _i, _i,
                            _i, _i, _i, _i64, _i, _p]),
    "rkv_gelu": (_i, [_p, _p, _i64, _p]),
    "rkv_add": (_i, [_p, _p, _p, _i64, _p]),
    "rkv_mul_scalar": (_i, [_p, _p, _f, _i64, _p]),
    "rkv_softmax_dim": (_i, [_p, _p, _i64, _i64, _i64, _p]),
    "rkv_matmul": (_i, [_p, _p, _p, _i, _i, _i, _p]),
    "rkv_transpose": (_i, [_p, _p, _i, _i, _p]),
    "rkv_argmax": (_i, [_p, _p, _i, _i, _p]),
    "rkv_decoder_param_count": (_i64, [_p]),
    "rkv_decoder_init_params": (_i, [_p, C.c_uint64, _f, _p]),
    "rkv_decoder_create": (_p, [_p, _p, _i64, _p]),
    "rkv_decoder_destroy": (None, [_p]),
    "rkv_decoder_generate": (_i, [_p, _p, _i, _i, _p, _p]),
    "rkv_decoder_load_safetensors": (_i, [_p, C.c_char_p, _p, _i64]),
    "rkv_decoder_save_safetensors": (_i, [_p, _p, _i64, C.c_char_p]),
    "rkv_decoder_load_safetensors_device": (_i, [_p, C.c_char_p]),
    "rkv_decoder_create_from_safetensors": (_p, [_p, C.c_char_p, _p]),
    "rkv_st_open": (_p, [C.c_char_p]),
    "rkv_st_close": (None, [_p]),
    "rkv_st_num_tensors": (_i64, [_p]),
    "rkv_st_tensor": (_i, [_p, _i64, C.POINTER(C.c_char_p), C.POINTER(C.c_char_p),
                           C.POINTER(C.c_int), _p, _i]),
    "rkv_st_load": (_i, [_p, _i, _p, _p, _p, _p, _i, _p]),
    "rkv_engine_create": (_p, [_p, _p, _i64, _i64, _i, _p]),
    "rkv_engine_destroy": (None, [_p]),
    "rkv_engine_submit": (_i64, [_p, _p, _i, _i, _i]),
    "rkv_engine_step": (_i, [_p]),
    "rkv_engine_run": (_i, [_p, _i]),
    "rkv_engine_scheduler": (_p, [_p]),
    "rkv_rng_raw": (_i, [C.c_uint64, _p, _i64]),
    "rkv_fill_normal": (_i, [_p, _i64, C.c_uint64, _f]),
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
