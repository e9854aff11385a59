"""numpy front end of the CPU oracle (oracle/rkv_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py, always as the checker or the timed CPU
baseline.  The product package ``rustral_amd`` never imports it.

Every wrapper takes and returns numpy arrays in the pool layout shared with
the GPU library: ``pool[num_blocks, Hkv, block_size, D]`` (float32, or uint16
holding bf16 bits).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

F32, BF16 = 0, 1
_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "liboracle.so")
_lib = None


def build() -> str:
    """Compile liboracle.so with the committed Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_p = C.c_void_p
_i32, _i64, _f32 = C.c_int32, C.c_int64, C.c_float


def _declare(L):
    L.orc_bf16_from_f32.restype = C.c_uint16
    L.orc_bf16_from_f32.argtypes = [_f32]
    L.orc_bf16_from_f32_array.argtypes = [_p, _p, _i64]
    L.orc_f32_from_bf16_array.argtypes = [_p, _p, _i64]
    L.orc_append.argtypes = [_p, _p, _p, _p, _p, _i64, C.c_int, C.c_int, C.c_int, _i64, _i64,
                             _i64, C.c_int]
    L.orc_gather.argtypes = [_p, _p, _p, _p, _p, C.c_int, _p, _p, C.c_int, C.c_int, C.c_int,
                             C.c_int, _i64, C.c_int, C.c_int, C.c_int]
    L.orc_copy_blocks.argtypes = [_p, _p, _i64, C.c_int, _p, C.c_int, _i64, _i64]
    L.orc_softmax_rows.argtypes = [_p, _p, C.c_int, C.c_int]
    L.orc_softmax_dim.restype = C.c_int
    L.orc_softmax_dim.argtypes = [_p, _p, _i64, _i64, _i64]
    L.orc_matmul.argtypes = [_p, _p, _p, C.c_int, C.c_int, C.c_int]
    L.orc_transpose.argtypes = [_p, _p, C.c_int, C.c_int]
    L.orc_mul_scalar.argtypes = [_p, _p, _f32, _i64]
    L.orc_argmax.restype = _i64
    L.orc_argmax.argtypes = [_p, _i64]
    dec = [_p, _p, _p, _p, _p, C.c_int, _p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _i64,
           _f32, C.c_int]
    L.orc_decode_attention.argtypes = dec
    L.orc_decode_attention_f64.argtypes = dec
    L.orc_decode_attention_mt.argtypes = dec + [C.c_int]
    L.orc_decode_partials.argtypes = [_p, _p] + dec + [C.c_int, C.c_int]
    L.orc_splitk_merge.argtypes = [_p, _p, _p, _p, _p, C.c_int, C.c_int, C.c_int, C.c_int,
                                   C.c_int, C.c_int, C.c_int]
    L.orc_e4m3_from_f32.restype = C.c_uint8
    L.orc_e4m3_from_f32.argtypes = [_f32]
    L.orc_f32_from_e4m3.restype = _f32
    L.orc_f32_from_e4m3.argtypes = [C.c_uint8]
    L.orc_quantize_row.argtypes = [_p, C.c_int, C.c_int, _p, _p]
    L.orc_append_q.argtypes = [_p, _p, _p, _p, _p, _p, _p, _i64, C.c_int, C.c_int, C.c_int, _i64,
                               _i64, _i64, C.c_int]
    L.orc_append_q.restype = C.c_int
    L.orc_dequantize_pool.argtypes = [_p, _p, _i64, C.c_int, C.c_int, _p]
    L.orc_prefill_attention.argtypes = [_p, _p, _p, _p, _p, C.c_int, _p, _p, C.c_int, C.c_int,
                                        C.c_int, C.c_int, C.c_int, _i64, _f32, C.c_int]
    L.orc_decoder_param_count.restype = _i64
    L.orc_decoder_param_count.argtypes = [_p]
    L.orc_linear.argtypes = [_p, _p, _p, _p, C.c_int, C.c_int, C.c_int]
    L.orc_layer_norm.argtypes = [_p, _p, _p, _p, C.c_int, C.c_int, _f32]
    L.orc_gelu.argtypes = [_p, _p, _i64]
    L.orc_positional_encoding.argtypes = [_p, C.c_int, C.c_int]
    L.orc_decoder_generate.argtypes = [_p, _p, _p, C.c_int, C.c_int, _p, _p]
    for name in ("orc_decoder_generate", "orc_append", "orc_gather", "orc_copy_blocks", "orc_decode_attention",
                 "orc_decode_attention_f64", "orc_decode_attention_mt", "orc_decode_partials",
                 "orc_splitk_merge", "orc_prefill_attention"):
        getattr(L, name).restype = C.c_int


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle wants C-contiguous arrays"
    return a.ctypes.data


def _check(rc: int, name: str):
    if rc != 0:
        raise ValueError(f"{name} rejected its arguments (rc={rc})")


def _dtype_code(pool: np.ndarray) -> int:
    if pool.dtype == np.float32:
        return F32
    if pool.dtype == np.uint16:
        return BF16
    raise TypeError(f"pool dtype {pool.dtype} (want float32 or uint16 bf16 bits)")


# ---- bf16 -------------------------------------------------------------------

def bf16_from_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().orc_bf16_from_f32_array(_ptr(x), _ptr(y), x.size)
    return y


def f32_from_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    y = np.empty(x.shape, dtype=np.float32)
    lib().orc_f32_from_bf16_array(_ptr(x), _ptr(y), x.size)
    return y


def pool_as_f32(pool: np.ndarray) -> np.ndarray:
    return pool if pool.dtype == np.float32 else f32_from_bf16(pool)


# ---- path functions ---------------------------------------------------------

def append(k_pool, v_pool, k_new, v_new, slot_mapping, *, tok_stride=None, head_stride=None):
    """In-place append; k_new/v_new are float32 with rows addressed by strides
    (defaults: [n_tokens, Hkv, D] contiguous)."""
    nb, hkv, bs, d = k_pool.shape
    n = slot_mapping.shape[0]
    tok_stride = hkv * d if tok_stride is None else tok_stride
    head_stride = d if head_stride is None else head_stride
    k_new = np.ascontiguousarray(k_new, dtype=np.float32)
    v_new = np.ascontiguousarray(v_new, dtype=np.float32)
    sm = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    _check(lib().orc_append(_ptr(k_pool), _ptr(v_pool), _ptr(k_new), _ptr(v_new), _ptr(sm), n,
                            hkv, d, bs, nb, tok_stride, head_stride, _dtype_code(k_pool)),
           "orc_append")


def gather(k_pool, v_pool, block_tables, ctx_lens, *, max_ctx=None, out_offsets=None,
           out_f32=False, k_out=None, v_out=None):
    nb, hkv, bs, d = k_pool.shape
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cl = np.ascontiguousarray(ctx_lens, dtype=np.int32)
    B, mbs = bt.shape
    pdt = _dtype_code(k_pool)
    odt = F32 if out_f32 else pdt
    np_dt = np.float32 if odt == F32 else np.uint16
    if out_offsets is None:
        max_ctx = int(max(1, cl.max(initial=0))) if max_ctx is None else max_ctx
        shape = (B, hkv, max_ctx, d)
    else:
        out_offsets = np.ascontiguousarray(out_offsets, dtype=np.int64)
        max_ctx = 0
        shape = (int(out_offsets[-1] + hkv * max(0, min(int(cl[-1]), mbs * bs)) * d),)
    if k_out is None:
        k_out = np.zeros(shape, dtype=np_dt)
        v_out = np.zeros(shape, dtype=np_dt)
    _check(lib().orc_gather(_ptr(k_out), _ptr(v_out), _ptr(k_pool), _ptr(v_pool), _ptr(bt), mbs,
                            _ptr(cl), _ptr(out_offsets), B, hkv, d, bs, nb, max_ctx, pdt, odt),
           "orc_gather")
    return k_out, v_out


def copy_blocks(k_pool, v_pool, pairs, *, n_layers=1, layer_stride_bytes=0, block_bytes=None,
                num_blocks=None):
    """In-place copy; k_pool/v_pool may be [n_layers, num_blocks, Hkv, BS, D] or
    [num_blocks, Hkv, BS, D]."""
    pr = np.ascontiguousarray(pairs, dtype=np.int32).reshape(-1, 2)
    if k_pool.ndim == 5:
        n_layers = k_pool.shape[0]
        layer_stride_bytes = k_pool[0].nbytes
        per = k_pool[0]
    else:
        per = k_pool
    nb = per.shape[0] if num_blocks is None else num_blocks
    bb = per[0].nbytes if block_bytes is None else block_bytes
    _check(lib().orc_copy_blocks(_ptr(k_pool), _ptr(v_pool), layer_stride_bytes, n_layers,
                                 _ptr(pr), pr.shape[0], bb, nb), "orc_copy_blocks")


def softmax_rows(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_softmax_rows(_ptr(x), _ptr(y), x.shape[0], x.shape[1])
    return y


def softmax_dim(x: np.ndarray, dim: int) -> np.ndarray:
    """CpuOps::softmax_dim of x along dim (any rank)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if not 0 <= dim < x.ndim:
        raise ValueError(f"softmax_dim: dim {dim} out of range for shape {x.shape}")
    outer = int(np.prod(x.shape[:dim], dtype=np.int64))
    inner = int(np.prod(x.shape[dim + 1:], dtype=np.int64))
    y = np.empty_like(x)
    if lib().orc_softmax_dim(_ptr(x), _ptr(y), outer, x.shape[dim], inner) != 0:
        raise ValueError("softmax_dim: axis size is 0")
    return y


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    (m, k), (k2, n) = a.shape, b.shape
    if k != k2:
        raise ValueError(f"matmul: inner sizes {k} and {k2} differ")
    y = np.empty((m, n), np.float32)
    lib().orc_matmul(_ptr(a), _ptr(b), _ptr(y), m, k, n)
    return y


def transpose(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty((x.shape[1], x.shape[0]), np.float32)
    lib().orc_transpose(_ptr(x), _ptr(y), x.shape[0], x.shape[1])
    return y


def mul_scalar(x: np.ndarray, s: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_mul_scalar(_ptr(x), _ptr(y), s, x.size)
    return y


def argmax(x) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().orc_argmax(_ptr(x), x.size))


def _dec_args(q, k_pool, v_pool, block_tables, ctx_lens, scale):
    nb, hkv, bs, d = k_pool.shape
    q = np.ascontiguousarray(q, dtype=np.float32)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cl = np.ascontiguousarray(ctx_lens, dtype=np.int32)
    B, hq, _ = q.shape
    return (q, bt, cl), [_ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(bt), bt.shape[1], _ptr(cl), B,
                         hq, hkv, d, bs, nb, float(scale), _dtype_code(k_pool)]


def decode_attention(q, k_pool, v_pool, block_tables, ctx_lens, scale, *, f64=False,
                     n_threads=0):
    keep, args = _dec_args(q, k_pool, v_pool, block_tables, ctx_lens, scale)
    out = np.zeros(keep[0].shape, dtype=np.float64 if f64 else np.float32)
    if f64:
        rc = lib().orc_decode_attention_f64(_ptr(out), *args)
    elif n_threads > 0:
        rc = lib().orc_decode_attention_mt(_ptr(out), *args, n_threads)
    else:
        rc = lib().orc_decode_attention(_ptr(out), *args)
    _check(rc, "orc_decode_attention")
    return out


def decode_splitk(q, k_pool, v_pool, block_tables, ctx_lens, scale, partition_size):
    """Two-pass split-K: partials per partition, then the online-softmax merge."""
    keep, args = _dec_args(q, k_pool, v_pool, block_tables, ctx_lens, scale)
    B, hq, d = keep[0].shape
    bs = k_pool.shape[2]
    mbs = keep[1].shape[1]
    max_parts = max(1, -(-mbs * bs // partition_size))
    m = np.zeros((B, hq, max_parts), np.float32)
    l = np.zeros_like(m)
    acc = np.zeros((B, hq, max_parts, d), np.float32)
    _check(lib().orc_decode_partials(_ptr(m), _ptr(l), _ptr(acc), *args, partition_size,
                                     max_parts), "orc_decode_partials")
    out = np.zeros((B, hq, d), np.float32)
    _check(lib().orc_splitk_merge(_ptr(out), _ptr(m), _ptr(l), _ptr(acc), _ptr(keep[2]), mbs, bs,
                                  B, hq, d, partition_size, max_parts), "orc_splitk_merge")
    return out, (m, l, acc)


I8, FP8 = 2, 3


def e4m3_from_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    return np.array([lib().orc_e4m3_from_f32(float(v)) for v in x], np.uint8)


def f32_from_e4m3(b) -> np.ndarray:
    b = np.ascontiguousarray(b, np.uint8).ravel()
    return np.array([lib().orc_f32_from_e4m3(int(v)) for v in b], np.float32)


def quantize_rows(x, dtype):
    """Quantizes each row of x [rows, n] -> (bytes [rows, n] uint8, scales [rows] fp32)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, n = x.shape
    q = np.zeros((rows, n), np.uint8)
    s = np.zeros(rows, np.float32)
    for r in range(rows):
        lib().orc_quantize_row(_ptr(x[r]), n, dtype, q[r].ctypes.data_as(C.c_void_p),
                               s[r:].ctypes.data_as(C.c_void_p))
    return q, s


def append_q(k_pool, v_pool, k_scale, v_scale, k_new, v_new, slot_mapping, dtype):
    """Quantizing append into uint8 pools [nb, Hkv, BS, D] and scales [nb, Hkv, BS]."""
    nb, hkv, bs, d = k_pool.shape
    k_new = np.ascontiguousarray(k_new, np.float32)
    v_new = np.ascontiguousarray(v_new, np.float32)
    sm = np.ascontiguousarray(slot_mapping, np.int64)
    _check(lib().orc_append_q(_ptr(k_pool), _ptr(v_pool), _ptr(k_scale), _ptr(v_scale),
                              _ptr(k_new), _ptr(v_new), _ptr(sm), len(sm), hkv, d, bs, nb,
                              hkv * d, d, dtype), "orc_append_q")


def dequantize_pool(pool, scales, dtype):
    """fp32 values of a 1-byte pool: byte value * its row's scale."""
    pool = np.ascontiguousarray(pool, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    d = pool.shape[-1]
    out = np.zeros(pool.shape, np.float32)
    lib().orc_dequantize_pool(_ptr(pool), _ptr(scales), pool.size // d, d, dtype, _ptr(out))
    return out


def prefill_attention(q, k_pool, v_pool, block_tables, q_start, ctx_lens, scale):
    """Causal prefill over the paged pool: q/out [total, Hq, D]; sequence b
    owns rows q_start[b] .. q_start[b+1]-1, at positions ctx_lens[b] - n_b + i."""
    nb, hkv, bs, d = k_pool.shape
    q = np.ascontiguousarray(q, dtype=np.float32)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    qs = np.ascontiguousarray(q_start, dtype=np.int32)
    cl = np.ascontiguousarray(ctx_lens, dtype=np.int32)
    total, hq, _ = q.shape
    assert qs[-1] <= total and len(qs) == len(cl) + 1
    out = np.zeros_like(q)
    _check(lib().orc_prefill_attention(_ptr(out), _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(bt),
                                       bt.shape[1], _ptr(qs), _ptr(cl), len(cl), hq, hkv, d, bs,
                                       nb, float(scale), _dtype_code(k_pool)),
           "orc_prefill_attention")
    return out


# ---- config-0 decoder ----------------------------------------------------------

class DecoderConfig(C.Structure):
    """orc_decoder_config (rkv_oracle.h); the same field order as the product's
    rkv_decoder_config."""
    _fields_ = [("vocab", C.c_int), ("d_model", C.c_int), ("n_heads", C.c_int),
                ("n_kv_heads", C.c_int), ("d_ff", C.c_int), ("n_layers", C.c_int),
                ("max_seq", C.c_int), ("eps", C.c_float)]


# benchmark configs[0]: 2 layers, d_model 128, 4 heads (head_dim 32), MLP 512,
# vocab 1000; 32 prompt ids + 64 greedy tokens = 96 positions.
CONFIG0 = dict(vocab=1000, d_model=128, n_heads=4, n_kv_heads=4, d_ff=512, n_layers=2,
               max_seq=128, eps=1e-5)


def decoder_config(**kw) -> DecoderConfig:
    d = dict(CONFIG0)
    d.update(kw)
    return DecoderConfig(**d)


def decoder_param_count(cfg: DecoderConfig) -> int:
    return int(lib().orc_decoder_param_count(C.byref(cfg)))


def linear(x, w, b=None):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    rows, in_dim = x.shape
    out_dim = w.shape[0]
    y = np.empty((rows, out_dim), np.float32)
    lib().orc_linear(_ptr(y), _ptr(x), _ptr(w),
                     None if b is None else _ptr(np.ascontiguousarray(b, np.float32)),
                     rows, in_dim, out_dim)
    return y


def layer_norm(x, g, b, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_layer_norm(_ptr(y), _ptr(x), _ptr(np.ascontiguousarray(g, np.float32)),
                         _ptr(np.ascontiguousarray(b, np.float32)), x.shape[0], x.shape[1], eps)
    return y


def gelu(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_gelu(_ptr(y), _ptr(x), x.size)
    return y


def positional_encoding(max_len, d_model):
    pe = np.empty((max_len, d_model), np.float32)
    lib().orc_positional_encoding(_ptr(pe), max_len, d_model)
    return pe


def decoder_generate(cfg: DecoderConfig, params, prompt, n_new, *, logits=False):
    params = np.ascontiguousarray(params, np.float32)
    assert params.size == decoder_param_count(cfg)
    prompt = np.ascontiguousarray(prompt, np.int32)
    toks = np.empty(n_new, np.int32)
    lg = np.empty((n_new, cfg.vocab), np.float32) if logits else None
    _check(lib().orc_decoder_generate(C.byref(cfg), _ptr(params), _ptr(prompt), len(prompt),
                                      n_new, _ptr(toks), _ptr(lg)), "orc_decoder_generate")
    return (toks, lg) if logits else toks
