"""The model glue around the paged-KV path: device TensorOps subset, the
greedy decoder of benchmark configs[0], and the seeded parameter generator
(include/rustral_model.h, implemented in csrc/model_ops.hip and
csrc/decoder.hip).
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import torch

from ._lib import RkvError, check, lib
from .kv import _dev, _dtype_code, _stream


class DecoderConfig(C.Structure):
    """rkv_decoder_config."""
    _fields_ = [("vocab", C.c_int), ("d_model", C.c_int), ("n_heads", C.c_int),
                ("n_kv_heads", C.c_int), ("d_ff", C.c_int), ("n_layers", C.c_int),
                ("max_seq", C.c_int), ("eps", C.c_float)]


# benchmark configs[0]: 2 layers, d_model 128, 4 heads x 32, MLP 512, vocab 1000.
CONFIG0 = dict(vocab=1000, d_model=128, n_heads=4, n_kv_heads=4, d_ff=512, n_layers=2,
               max_seq=128, eps=1e-5)


def config(**kw) -> DecoderConfig:
    d = dict(CONFIG0)
    d.update(kw)
    return DecoderConfig(**d)


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def param_count(cfg: DecoderConfig) -> int:
    n = lib().rkv_decoder_param_count(C.byref(cfg))
    if n < 0:
        raise ValueError("invalid decoder configuration")
    return int(n)


def init_params(cfg: DecoderConfig, seed: int = 0, std: float = 0.02) -> np.ndarray:
    """Random parameters: N(0, std^2) weights in parameter order from one
    seeded stream, unit layer-norm gains, zero biases."""
    out = np.empty(param_count(cfg), np.float32)
    check(lib().rkv_decoder_init_params(C.byref(cfg), seed, std, _p(out)))
    return out


def load_safetensors(cfg: DecoderConfig, path: str) -> np.ndarray:
    """Parameters from a safetensors file (strict: exactly the decoder's names,
    shapes and F32), in the packed order rkv_decoder_create takes."""
    out = np.empty(param_count(cfg), np.float32)
    check(lib().rkv_decoder_load_safetensors(C.byref(cfg), str(path).encode(), _p(out), out.size))
    return out


def save_safetensors(cfg: DecoderConfig, params: np.ndarray, path: str) -> None:
    params = np.ascontiguousarray(params, np.float32)
    check(lib().rkv_decoder_save_safetensors(C.byref(cfg), _p(params), params.size,
                                             str(path).encode()))


def rng_raw(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint64)
    check(lib().rkv_rng_raw(seed, _p(out), n))
    return out


def fill_normal(n: int, seed: int, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    check(lib().rkv_fill_normal(_p(out), n, seed, std))
    return out


class SafetensorsFile:
    """A memory-mapped safetensors file (rkv_st_*): its entries, and the
    strict load of the reference's load_model into host arrays or device
    tensors."""

    def __init__(self, path):
        h = lib().rkv_st_open(str(path).encode())
        if not h:
            raise RkvError(-1, lib().rkv_last_error().decode())
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            lib().rkv_st_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the module is torn down
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def entries(self) -> dict:
        """name -> (dtype, shape) in header order."""
        out = {}
        for i in range(lib().rkv_st_num_tensors(self._h)):
            name, dt, nd = C.c_char_p(), C.c_char_p(), C.c_int()
            shape = (C.c_int64 * 8)()
            check(lib().rkv_st_tensor(self._h, i, C.byref(name), C.byref(dt), C.byref(nd),
                                      C.cast(shape, C.c_void_p), 8))
            out[name.value.decode()] = (dt.value.decode(), tuple(shape[:nd.value]))
        return out

    def load(self, dsts: dict) -> None:
        """Strict load (every name of the file, F32, equal shapes) into the
        given destinations: name -> float32 numpy array (host) or contiguous
        float32 device tensor; all of one kind."""
        names = list(dsts)
        on_dev = [isinstance(dsts[n], torch.Tensor) for n in names]
        if any(on_dev) and not all(on_dev):
            raise ValueError("destinations must be all host arrays or all device tensors")
        dev = bool(names) and on_dev[0]
        ptrs, dims, shapes = [], [], []
        for n in names:
            t = dsts[n]
            if dev:
                _dev(t, n, torch.float32)
                ptrs.append(t.data_ptr())
            else:
                if t.dtype != np.float32 or not t.flags["C_CONTIGUOUS"] or not t.flags["WRITEABLE"]:
                    raise ValueError(f"{n}: host destination must be a writable contiguous float32 array")
                ptrs.append(t.ctypes.data)
            dims.append(t.dim() if dev else t.ndim)
            shapes.extend(int(x) for x in t.shape)
        c_names = (C.c_char_p * max(1, len(names)))(*[n.encode() for n in names])
        c_dims = (C.c_int * max(1, len(dims)))(*dims)
        c_shapes = (C.c_int64 * max(1, len(shapes)))(*shapes)
        c_ptrs = (C.c_void_p * max(1, len(ptrs)))(*ptrs)
        stream = torch.cuda.current_stream(dsts[names[0]].device).cuda_stream if dev else None
        check(lib().rkv_st_load(self._h, len(names), C.cast(c_names, C.c_void_p),
                                C.cast(c_dims, C.c_void_p), C.cast(c_shapes, C.c_void_p),
                                C.cast(c_ptrs, C.c_void_p), int(dev), stream))


class Decoder:
    """Greedy decoder on the current device (rkv_decoder_*)."""

    def __init__(self, cfg: DecoderConfig, params: np.ndarray | None = None, device=None, *,
                 path=None):
        """params: the packed host parameter array; or path: a safetensors file
        loaded strictly straight into device memory."""
        if (params is None) == (path is None):
            raise ValueError("give exactly one of params and path")
        dev = torch.device("cuda:0") if device is None else torch.device(device)
        self._stream = torch.cuda.current_stream(dev).cuda_stream
        self.cfg = cfg
        if path is not None:
            h = lib().rkv_decoder_create_from_safetensors(C.byref(cfg), str(path).encode(),
                                                          self._stream)
        else:
            params = np.ascontiguousarray(params, np.float32)
            h = lib().rkv_decoder_create(C.byref(cfg), _p(params), params.size, self._stream)
        if not h:
            raise RkvError(-1, lib().rkv_last_error().decode())
        self._h = h

    def load_safetensors(self, path) -> None:
        """Replaces the parameters with a safetensors file's (strict load
        straight into the decoder's device memory)."""
        check(lib().rkv_decoder_load_safetensors_device(self._h, str(path).encode()))

    def __del__(self):
        if getattr(self, "_h", None):
            try:
                lib().rkv_decoder_destroy(self._h)
            except Exception:  # interpreter shutdown: the module is torn down
                pass
            self._h = None

    def generate(self, prompt, n_new: int, *, logits: bool = False):
        prompt = np.ascontiguousarray(prompt, np.int32)
        toks = np.empty(max(n_new, 1), np.int32)
        lg = np.empty((max(n_new, 1), self.cfg.vocab), np.float32) if logits else None
        check(lib().rkv_decoder_generate(self._h, _p(prompt), len(prompt), n_new, _p(toks),
                                         None if lg is None else _p(lg)))
        toks = toks[:n_new]
        return (toks, lg[:n_new]) if logits else toks


class Engine:
    """Continuous-batching serving engine on the current device (rkv_engine_*):
    the scheduler's batch runs through the decoder each step."""

    def __init__(self, cfg: DecoderConfig, params: np.ndarray, num_blocks: int,
                 max_batch_size: int = 8, device=None):
        from .serving import Scheduler
        params = np.ascontiguousarray(params, np.float32)
        dev = torch.device("cuda:0") if device is None else torch.device(device)
        self._stream = torch.cuda.current_stream(dev).cuda_stream
        self.cfg = cfg
        h = lib().rkv_engine_create(C.byref(cfg), _p(params), params.size, num_blocks,
                                    max_batch_size, self._stream)
        if not h:
            raise RkvError(-1, lib().rkv_last_error().decode())
        self._h = h
        self.scheduler = Scheduler._borrow(lib().rkv_engine_scheduler(h), self)

    def __del__(self):
        if getattr(self, "_h", None):
            self.scheduler = None
            try:
                lib().rkv_engine_destroy(self._h)
            except Exception:  # interpreter shutdown: the module is torn down
                pass
            self._h = None

    def submit(self, prompt, max_tokens: int, priority: int = 1) -> int:
        prompt = np.ascontiguousarray(prompt, np.int32)
        rid = lib().rkv_engine_submit(self._h, _p(prompt), len(prompt), max_tokens, priority)
        if rid < 0:
            check(int(rid))
        return int(rid)

    def step(self) -> int:
        n = lib().rkv_engine_step(self._h)
        if n < 0:
            check(n)
        return n

    def run(self, max_steps: int = 1 << 30) -> int:
        n = lib().rkv_engine_run(self._h, max_steps)
        if n < 0:
            check(n)
        return n

    def generated(self, request_id: int) -> list[int]:
        return self.scheduler.generated(request_id)


# ---- device ops on torch tensors ---------------------------------------------------

def linear(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None = None) -> torch.Tensor:
    _dev(x, "x", torch.float32), _dev(w, "w", torch.float32)
    rows, in_dim = x.shape
    out_dim = w.shape[0]
    y = torch.empty((rows, out_dim), dtype=torch.float32, device=x.device)
    check(lib().rkv_linear(y.data_ptr(), x.data_ptr(), w.data_ptr(),
                           None if b is None else _dev(b, "b", torch.float32).data_ptr(),
                           rows, in_dim, out_dim, _stream(x)))
    return y


def layer_norm(x: torch.Tensor, g: torch.Tensor, b: torch.Tensor, eps: float = 1e-5):
    _dev(x, "x", torch.float32)
    y = torch.empty_like(x)
    check(lib().rkv_layer_norm(y.data_ptr(), x.data_ptr(), g.data_ptr(), b.data_ptr(),
                               x.shape[0], x.shape[1], eps, _stream(x)))
    return y


def qkv_append(x: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor, wv: torch.Tensor,
               k_pool: torch.Tensor, v_pool: torch.Tensor, slot_mapping: torch.Tensor,
               bq: torch.Tensor | None = None, bk: torch.Tensor | None = None,
               bv: torch.Tensor | None = None, ln_g: torch.Tensor | None = None,
               ln_b: torch.Tensor | None = None, eps: float = 1e-5) -> torch.Tensor:
    """LN1 (when ln_g / ln_b are given), q / k / v projections and the KV
    append of one layer in one launch; returns q [n_tokens, q_dim].  The pools
    ([num_blocks, Hkv, BS, D], float32 or bfloat16) receive k and v at
    slot_mapping (int64 [n_tokens], < 0: skip)."""
    _dev(x, "x", torch.float32), _dev(slot_mapping, "slot_mapping", torch.int64)
    for name, w in (("wq", wq), ("wk", wk), ("wv", wv)):
        _dev(w, name, torch.float32)
    _dev(k_pool, "k_pool"), _dev(v_pool, "v_pool")
    n_tok, d_model = x.shape
    nb, hkv, bs, hd = k_pool.shape
    if v_pool.shape != k_pool.shape or v_pool.dtype != k_pool.dtype:
        raise ValueError("K and V pools differ")
    if wq.shape[1] != d_model or wk.shape != (hkv * hd, d_model) or wv.shape != wk.shape:
        raise ValueError("projection shapes do not match x and the pools")
    if slot_mapping.shape != (n_tok,):
        raise ValueError("slot_mapping must be [n_tokens]")
    if (ln_g is None) != (ln_b is None):
        raise ValueError("ln_g and ln_b are given together")
    q = torch.empty((n_tok, wq.shape[0]), dtype=torch.float32, device=x.device)
    opt = lambda t, n: None if t is None else _dev(t, n, torch.float32).data_ptr()  # noqa: E731
    check(lib().rkv_qkv_append(q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(),
                               slot_mapping.data_ptr(), x.data_ptr(), opt(ln_g, "ln_g"),
                               opt(ln_b, "ln_b"), eps, wq.data_ptr(), opt(bq, "bq"),
                               wk.data_ptr(), opt(bk, "bk"), wv.data_ptr(), opt(bv, "bv"),
                               n_tok, d_model, wq.shape[0], hkv, hd, bs, nb,
                               _dtype_code(k_pool), _stream(x)))
    return q


def gelu(x: torch.Tensor) -> torch.Tensor:
    _dev(x, "x", torch.float32)
    y = torch.empty_like(x)
    check(lib().rkv_gelu(y.data_ptr(), x.data_ptr(), x.numel(), _stream(x)))
    return y


def add(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    _dev(a, "a", torch.float32), _dev(b, "b", torch.float32)
    y = torch.empty_like(a)
    check(lib().rkv_add(y.data_ptr(), a.data_ptr(), b.data_ptr(), a.numel(), _stream(a)))
    return y


def mul_scalar(x: torch.Tensor, s: float) -> torch.Tensor:
    _dev(x, "x", torch.float32)
    y = torch.empty_like(x)
    check(lib().rkv_mul_scalar(y.data_ptr(), x.data_ptr(), s, x.numel(), _stream(x)))
    return y


def softmax_dim(x: torch.Tensor, dim: int) -> torch.Tensor:
    """TensorOps::softmax_dim: softmax of x along dim (any rank; contiguous)."""
    _dev(x, "x", torch.float32)
    if not 0 <= dim < x.dim():
        raise ValueError(f"softmax_dim: dim {dim} out of range for shape {tuple(x.shape)}")
    outer = math.prod(x.shape[:dim])
    inner = math.prod(x.shape[dim + 1:])
    y = torch.empty_like(x)
    check(lib().rkv_softmax_dim(y.data_ptr(), x.data_ptr(), outer, x.shape[dim], inner,
                                _stream(x)))
    return y


def matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    _dev(a, "a", torch.float32), _dev(b, "b", torch.float32)
    (m, k), (k2, n) = a.shape, b.shape
    if k != k2:
        raise ValueError(f"matmul: inner sizes {k} and {k2} differ")
    y = torch.empty((m, n), dtype=torch.float32, device=a.device)
    check(lib().rkv_matmul(y.data_ptr(), a.data_ptr(), b.data_ptr(), m, k, n, _stream(a)))
    return y


def transpose(x: torch.Tensor) -> torch.Tensor:
    _dev(x, "x", torch.float32)
    m, n = x.shape
    y = torch.empty((n, m), dtype=torch.float32, device=x.device)
    check(lib().rkv_transpose(y.data_ptr(), x.data_ptr(), m, n, _stream(x)))
    return y


def argmax(x: torch.Tensor) -> torch.Tensor:
    _dev(x, "x", torch.float32)
    rows, n = x.shape
    out = torch.empty(rows, dtype=torch.int32, device=x.device)
    check(lib().rkv_argmax(out.data_ptr(), x.data_ptr(), rows, n, _stream(x)))
    return out


def embed(table: torch.Tensor, ids: torch.Tensor, pe: torch.Tensor | None = None,
          positions: torch.Tensor | None = None) -> torch.Tensor:
    _dev(table, "table", torch.float32), _dev(ids, "ids", torch.int32)
    vocab, dim = table.shape
    out = torch.empty((ids.numel(), dim), dtype=torch.float32, device=table.device)
    check(lib().rkv_embed(out.data_ptr(), table.data_ptr(), ids.data_ptr(),
                          None if pe is None else pe.data_ptr(),
                          None if positions is None else positions.data_ptr(), ids.numel(), vocab,
                          dim, 0 if pe is None else pe.shape[0], _stream(table)))
    return out


__all__ = ["DecoderConfig", "CONFIG0", "config", "param_count", "init_params", "rng_raw",
           "fill_normal", "Decoder", "linear", "layer_norm", "qkv_append", "gelu", "add", "argmax",
           "embed", "mul_scalar", "softmax_dim", "matmul", "transpose"]
