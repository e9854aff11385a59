"""torch-tensor front end of the paged-KV C ABI.

Device memory and streams come from PyTorch; every computation is one call
into librustral_kv.so on the tensor's current HIP stream.  Pools are
``[num_blocks, Hkv, block_size, D]`` (or ``[n_layers, num_blocks, Hkv,
block_size, D]`` for multi-layer append/copy) in float32 or bfloat16.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from ._lib import RKV_BF16, RKV_F32, check, lib


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return RKV_F32
    if t.dtype == torch.bfloat16:
        return RKV_BF16
    raise TypeError(f"KV pool dtype {t.dtype}: want float32 or bfloat16")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _dev(t: torch.Tensor, name: str, dtype=None) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def check_attention_shapes(q_shape, pool_shape, tables_shape, lens_shape,
                           q_start_shape=None) -> None:
    """The shapes an attention call's kernels index by, checked before any
    launch: q [rows, Hq, D] with D the pool's head_dim and Hq a multiple of
    its KV heads; one block-table row and one length per sequence; q rows one
    per sequence (decode) or q_start of B + 1 offsets (prefill).  The kernels
    take sizes, not buffer lengths, so a mismatch would read past the tables
    or write rows of the wrong width into the pools."""
    hkv, d = pool_shape[1], pool_shape[3]
    if len(q_shape) != 3 or len(tables_shape) != 2 or len(lens_shape) != 1:
        raise ValueError("q, block_tables and ctx_lens must be rank 3, 2 and 1")
    if q_shape[2] != d:
        raise ValueError(f"q head_dim {q_shape[2]} does not match the pool's {d}")
    if q_shape[1] == 0 or q_shape[1] % hkv:
        raise ValueError(f"{q_shape[1]} query heads are not a multiple of {hkv} KV heads")
    seqs = lens_shape[0]
    if tables_shape[0] != seqs:
        raise ValueError(f"{tables_shape[0]} block-table rows for {seqs} sequences")
    if q_start_shape is None:
        if q_shape[0] != seqs:
            raise ValueError(f"{q_shape[0]} q rows for {seqs} sequences")
    elif tuple(q_start_shape) != (seqs + 1,):
        raise ValueError(f"q_start must hold {seqs + 1} offsets")


def append(k_pool: torch.Tensor, v_pool: torch.Tensor, k_new: torch.Tensor,
           v_new: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Scatter new K/V rows into the pools (every layer in one launch).

    k_pool/v_pool: [num_blocks, Hkv, BS, D] or [n_layers, num_blocks, Hkv, BS, D].
    k_new/v_new:   float32 [n_tokens, Hkv, D] or [n_layers, n_tokens, Hkv, D].
    slot_mapping:  int64 [n_tokens], slot = block * BS + row (< 0: skip).
    """
    _dev(k_pool, "k_pool"), _dev(v_pool, "v_pool")
    _dev(k_new, "k_new", torch.float32), _dev(v_new, "v_new", torch.float32)
    _dev(slot_mapping, "slot_mapping", torch.int64)
    multi = k_pool.dim() == 5
    n_layers = k_pool.shape[0] if multi else 1
    nb, hkv, bs, d = k_pool.shape[-4:]
    if k_new.shape != v_new.shape or k_pool.shape != v_pool.shape:
        raise ValueError("K and V shapes differ")
    if k_new.shape[-2:] != (hkv, d) or k_new.dim() != (4 if multi else 3):
        raise ValueError(f"k_new shape {tuple(k_new.shape)} does not match pool {tuple(k_pool.shape)}")
    n_tok = k_new.shape[-3]
    if slot_mapping.shape != (n_tok,):
        raise ValueError("slot_mapping must be [n_tokens]")
    if multi and k_new.shape[0] != n_layers:
        raise ValueError("k_new must have one slice per pool layer")
    pool_ls = nb * hkv * bs * d if multi else 0
    src_ls = n_tok * hkv * d if multi else 0
    check(lib().rkv_append(k_pool.data_ptr(), v_pool.data_ptr(), pool_ls, k_new.data_ptr(),
                           v_new.data_ptr(), src_ls, hkv * d, d, slot_mapping.data_ptr(), n_tok,
                           n_layers, hkv, d, bs, nb, _dtype_code(k_pool), _stream(k_pool)))


def gather(k_pool: torch.Tensor, v_pool: torch.Tensor, block_tables: torch.Tensor,
           ctx_lens: torch.Tensor, *, max_ctx: int | None = None,
           out_offsets: torch.Tensor | None = None, out_total: int | None = None,
           out_dtype: torch.dtype | None = None, k_out=None, v_out=None):
    """Reconstruct contiguous per-sequence K/V (KVCache layout [Hkv, L, D]).

    Padded: returns [B, Hkv, max_ctx, D].  Packed (out_offsets int64 [B] given):
    returns flat tensors of out_total elements.  Untouched rows keep the
    contents of k_out/v_out (zeros when allocated here).
    """
    _dev(k_pool, "k_pool"), _dev(v_pool, "v_pool")
    _dev(block_tables, "block_tables", torch.int32), _dev(ctx_lens, "ctx_lens", torch.int32)
    nb, hkv, bs, d = k_pool.shape
    B, mbs = block_tables.shape
    out_dtype = k_pool.dtype if out_dtype is None else out_dtype
    if out_offsets is None:
        if max_ctx is None:
            max_ctx = mbs * bs
        shape = (B, hkv, max_ctx, d)
        off_ptr = None
    else:
        _dev(out_offsets, "out_offsets", torch.int64)
        if out_total is None:
            raise ValueError("packed gather needs out_total")
        shape = (out_total,)
        off_ptr = out_offsets.data_ptr()
        max_ctx = 0
    if k_out is None:
        k_out = torch.zeros(shape, dtype=out_dtype, device=k_pool.device)
        v_out = torch.zeros(shape, dtype=out_dtype, device=k_pool.device)
    check(lib().rkv_gather(k_out.data_ptr(), v_out.data_ptr(), k_pool.data_ptr(),
                           v_pool.data_ptr(), block_tables.data_ptr(), mbs, ctx_lens.data_ptr(),
                           off_ptr, B, hkv, d, bs, nb, max_ctx, _dtype_code(k_pool),
                           _dtype_code(k_out), _stream(k_pool)))
    return k_out, v_out


def copy_blocks(k_pool: torch.Tensor, v_pool: torch.Tensor, pairs: torch.Tensor) -> None:
    """Block pairs[i,1] := block pairs[i,0] in every layer of the pools.

    pairs: int32 [n_pairs, 2] on the device; destinations must not be sources.
    """
    _dev(k_pool, "k_pool"), _dev(v_pool, "v_pool"), _dev(pairs, "pairs", torch.int32)
    multi = k_pool.dim() == 5
    n_layers = k_pool.shape[0] if multi else 1
    per = k_pool[0] if multi else k_pool
    nb = per.shape[0]
    block_bytes = per[0].numel() * per.element_size()
    layer_stride = per.numel() * per.element_size() if multi else 0
    check(lib().rkv_copy_blocks(k_pool.data_ptr(), v_pool.data_ptr(), layer_stride, n_layers,
                                pairs.data_ptr(), pairs.shape[0], block_bytes, nb,
                                _stream(k_pool)))


def workspace_bytes(num_seqs: int, num_q_heads: int, head_dim: int, max_context: int,
                    partition_size: int = 0) -> int:
    return int(lib().rkv_decode_workspace_bytes(num_seqs, num_q_heads, head_dim, max_context,
                                                partition_size))


def partition_size(dtype_code: int, max_context: int, requested: int = 0, head_dim: int = 128) -> int:
    """The partition size of the split entry points (a request <= 0: 640)."""
    p = lib().rkv_decode_partition_size(requested, head_dim, dtype_code, max_context)
    check(min(p, 0))
    return int(p)


def partition_size_for(num_seqs: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                       dtype_code: int, max_context: int, requested: int = 0) -> int:
    """The partition size decode_attention uses for a call of this shape (a
    request <= 0: the library's pick)."""
    p = lib().rkv_decode_partition_size_for(requested, num_seqs, num_q_heads, num_kv_heads,
                                            head_dim, dtype_code, max_context)
    check(min(p, 0))
    return int(p)


def decode_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                     block_tables: torch.Tensor, ctx_lens: torch.Tensor,
                     scale: float | None = None, *, max_context: int | None = None,
                     out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                     passes: str = "both", partition_size: int = 0) -> torch.Tensor:
    """Paged GQA decode attention: q [B, Hq, D] fp32 -> out [B, Hq, D] fp32.

    passes: "both" (default), "partitions" or "merge" (the two launches of
    the split-K algorithm, for callers that time or schedule them apart).
    partition_size: tokens per split-K partition (a multiple of 64 up to
    640; 0: the library's default for max_context).
    """
    _dev(q, "q", torch.float32), _dev(k_pool, "k_pool"), _dev(v_pool, "v_pool")
    _dev(block_tables, "block_tables", torch.int32), _dev(ctx_lens, "ctx_lens", torch.int32)
    nb, hkv, bs, d = k_pool.shape
    check_attention_shapes(q.shape, k_pool.shape, block_tables.shape, ctx_lens.shape)
    B, hq, dq = q.shape
    mbs = block_tables.shape[1]
    if max_context is None:
        max_context = mbs * bs
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if out is None:
        out = torch.empty_like(q)
    need = workspace_bytes(B, hq, d, max_context, partition_size)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_len = workspace.numel() * workspace.element_size() if workspace is not None else 0
    dt = _dtype_code(k_pool)
    s = _stream(q)
    if passes != "both" and partition_size <= 0:
        # the split entry points take 640 for 0: ask for this shape's pick so
        # the two passes partition like the one-call entry point
        partition_size = partition_size_for(B, hq, hkv, d, dt, min(max_context, mbs * bs))
    if passes in ("both", "partitions"):
        fn = lib().rkv_decode_attention if passes == "both" else lib().rkv_decode_attention_partitions
        check(fn(out.data_ptr(), q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(),
                 block_tables.data_ptr(), mbs, ctx_lens.data_ptr(), B, hq, hkv, d, bs, nb,
                 max_context, float(scale), dt, partition_size, ws_ptr, ws_len, s))
    elif passes == "merge":
        check(lib().rkv_decode_attention_merge(out.data_ptr(), ctx_lens.data_ptr(), mbs, B, hq, d,
                                               bs, max_context, dt, partition_size, ws_ptr, ws_len,
                                               s))
    else:
        raise ValueError(f"passes={passes!r}")
    return out


def decode_attention_append(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                            k_new: torch.Tensor, v_new: torch.Tensor, block_tables: torch.Tensor,
                            ctx_lens: torch.Tensor, scale: float | None = None, *,
                            max_context: int | None = None, out: torch.Tensor | None = None,
                            workspace: torch.Tensor | None = None,
                            partition_size: int = 0) -> torch.Tensor:
    """One decode step's append fused into decode_attention (bf16 pools).

    k_new, v_new: [B, Hkv, D] fp32, the rows of position ctx_lens[b] - 1
    (ctx_lens already counts the new token).  Writes them into the pools and
    returns what append followed by decode_attention returns.
    """
    _dev(q, "q", torch.float32), _dev(k_pool, "k_pool", torch.bfloat16)
    _dev(v_pool, "v_pool", torch.bfloat16)
    _dev(k_new, "k_new", torch.float32), _dev(v_new, "v_new", torch.float32)
    _dev(block_tables, "block_tables", torch.int32), _dev(ctx_lens, "ctx_lens", torch.int32)
    nb, hkv, bs, d = k_pool.shape
    check_attention_shapes(q.shape, k_pool.shape, block_tables.shape, ctx_lens.shape)
    B, hq, dq = q.shape
    if tuple(k_new.shape) != (B, hkv, d) or tuple(v_new.shape) != (B, hkv, d):
        raise ValueError("q, k_new and v_new must be [B, Hq, D], [B, Hkv, D], [B, Hkv, D]")
    mbs = block_tables.shape[1]
    if max_context is None:
        max_context = mbs * bs
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if out is None:
        out = torch.empty_like(q)
    need = workspace_bytes(B, hq, d, max_context, partition_size)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_len = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(lib().rkv_decode_attention_append(
        out.data_ptr(), q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), k_new.data_ptr(),
        v_new.data_ptr(), block_tables.data_ptr(), mbs, ctx_lens.data_ptr(), B, hq, hkv, d, bs,
        nb, max_context, float(scale), _lib.RKV_BF16, partition_size, ws_ptr, ws_len,
        _stream(q)))
    return out


_QFMT = {"int8": _lib.RKV_I8, "fp8": _lib.RKV_FP8, _lib.RKV_I8: _lib.RKV_I8,
         _lib.RKV_FP8: _lib.RKV_FP8}


def _qcode(fmt) -> int:
    if fmt not in _QFMT:
        raise ValueError(f"1-byte format {fmt!r}: want 'int8' or 'fp8'")
    return _QFMT[fmt]


def append_q(k_pool: torch.Tensor, v_pool: torch.Tensor, k_scale: torch.Tensor,
             v_scale: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
             slot_mapping: torch.Tensor, fmt: str = "int8") -> None:
    """Quantizing append into 1-byte pools (uint8 [.., nb, Hkv, BS, D]) with
    per-row fp32 scales ([.., nb, Hkv, BS]); fmt 'int8' or 'fp8' (OCP e4m3)."""
    _dev(k_pool, "k_pool", torch.uint8), _dev(v_pool, "v_pool", torch.uint8)
    _dev(k_scale, "k_scale", torch.float32), _dev(v_scale, "v_scale", torch.float32)
    _dev(k_new, "k_new", torch.float32), _dev(v_new, "v_new", torch.float32)
    _dev(slot_mapping, "slot_mapping", torch.int64)
    multi = k_pool.dim() == 5
    n_layers = k_pool.shape[0] if multi else 1
    nb, hkv, bs, d = k_pool.shape[-4:]
    if k_scale.shape != k_pool.shape[:-1] or v_scale.shape != v_pool.shape[:-1]:
        raise ValueError("scale pools must be the byte pools' shape without head_dim")
    n_tok = k_new.shape[-3]
    if slot_mapping.shape != (n_tok,) or k_new.shape[-2:] != (hkv, d):
        raise ValueError("k_new / slot_mapping shapes do not match the pool")
    pool_ls = nb * hkv * bs * d if multi else 0
    src_ls = n_tok * hkv * d if multi else 0
    check(lib().rkv_append_q(k_pool.data_ptr(), v_pool.data_ptr(), k_scale.data_ptr(),
                             v_scale.data_ptr(), pool_ls, k_new.data_ptr(), v_new.data_ptr(),
                             src_ls, hkv * d, d, slot_mapping.data_ptr(), n_tok, n_layers, hkv,
                             d, bs, nb, _qcode(fmt), _stream(k_pool)))


def gather_q(k_pool: torch.Tensor, v_pool: torch.Tensor, k_scale: torch.Tensor,
             v_scale: torch.Tensor, block_tables: torch.Tensor, ctx_lens: torch.Tensor,
             fmt: str = "int8", *, max_ctx: int | None = None,
             out_offsets: torch.Tensor | None = None, out_total: int | None = None,
             k_out=None, v_out=None) -> tuple[torch.Tensor, torch.Tensor]:
    """Dequantized K/V per sequence in fp32: padded [B, Hkv, max_ctx, D], or
    packed (out_offsets int64 [B] given) as flat tensors of out_total
    elements.  Untouched rows keep the contents of k_out/v_out (zeros when
    allocated here)."""
    _dev(k_pool, "k_pool", torch.uint8), _dev(v_pool, "v_pool", torch.uint8)
    _dev(k_scale, "k_scale", torch.float32), _dev(v_scale, "v_scale", torch.float32)
    _dev(block_tables, "block_tables", torch.int32), _dev(ctx_lens, "ctx_lens", torch.int32)
    nb, hkv, bs, d = k_pool.shape
    B, mbs = block_tables.shape
    if out_offsets is None:
        if max_ctx is None:
            max_ctx = mbs * bs
        shape = (B, hkv, max_ctx, d)
        off_ptr = None
    else:
        _dev(out_offsets, "out_offsets", torch.int64)
        if out_total is None:
            raise ValueError("packed gather needs out_total")
        shape = (out_total,)
        off_ptr = out_offsets.data_ptr()
        max_ctx = 0
    if k_out is None:
        k_out = torch.zeros(shape, dtype=torch.float32, device=k_pool.device)
        v_out = torch.zeros(shape, dtype=torch.float32, device=k_pool.device)
    _dev(k_out, "k_out", torch.float32), _dev(v_out, "v_out", torch.float32)
    if k_out.numel() < math.prod(shape) or v_out.numel() < math.prod(shape):
        raise ValueError("gather_q output smaller than the layout needs")
    check(lib().rkv_gather_q(k_out.data_ptr(), v_out.data_ptr(), k_pool.data_ptr(),
                             v_pool.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
                             block_tables.data_ptr(), mbs, ctx_lens.data_ptr(), off_ptr, B, hkv, d,
                             bs, nb, max_ctx, _qcode(fmt), _stream(k_pool)))
    return k_out, v_out


def decode_attention_append_q(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                              k_scale: torch.Tensor, v_scale: torch.Tensor, k_new: torch.Tensor,
                              v_new: torch.Tensor, block_tables: torch.Tensor,
                              ctx_lens: torch.Tensor, scale: float | None = None,
                              fmt: str = "int8", *, max_context: int | None = None,
                              out: torch.Tensor | None = None,
                              workspace: torch.Tensor | None = None,
                              partition_size: int = 0) -> torch.Tensor:
    """decode_attention_append over 1-byte pools: the new rows quantized as
    append_q quantizes them, then decode_attention_q, in one launch."""
    _dev(q, "q", torch.float32), _dev(k_pool, "k_pool", torch.uint8)
    _dev(v_pool, "v_pool", torch.uint8), _dev(k_scale, "k_scale", torch.float32)
    _dev(v_scale, "v_scale", torch.float32)
    _dev(k_new, "k_new", torch.float32), _dev(v_new, "v_new", torch.float32)
    _dev(block_tables, "block_tables", torch.int32), _dev(ctx_lens, "ctx_lens", torch.int32)
    nb, hkv, bs, d = k_pool.shape
    check_attention_shapes(q.shape, k_pool.shape, block_tables.shape, ctx_lens.shape)
    B, hq, dq = q.shape
    if tuple(k_new.shape) != (B, hkv, d) or tuple(v_new.shape) != (B, hkv, d):
        raise ValueError("q, k_new and v_new must be [B, Hq, D], [B, Hkv, D], [B, Hkv, D]")
    mbs = block_tables.shape[1]
    if max_context is None:
        max_context = mbs * bs
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if out is None:
        out = torch.empty_like(q)
    need = workspace_bytes(B, hq, d, max_context, partition_size)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_len = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(lib().rkv_decode_attention_append_q(
        out.data_ptr(), q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), k_scale.data_ptr(),
        v_scale.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), block_tables.data_ptr(), mbs,
        ctx_lens.data_ptr(), B, hq, hkv, d, bs, nb, max_context, float(scale), _qcode(fmt),
        partition_size, ws_ptr, ws_len, _stream(q)))
    return out


def decode_attention_q(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                       k_scale: torch.Tensor, v_scale: torch.Tensor, block_tables: torch.Tensor,
                       ctx_lens: torch.Tensor, scale: float | None = None, fmt: str = "int8", *,
                       max_context: int | None = None, out: torch.Tensor | None = None,
                       workspace: torch.Tensor | None = None, partition_size: int = 0) -> torch.Tensor:
    """decode_attention over 1-byte pools with per-row scales."""
    _dev(q, "q", torch.float32), _dev(k_pool, "k_pool", torch.uint8)
    _dev(v_pool, "v_pool", torch.uint8), _dev(k_scale, "k_scale", torch.float32)
    _dev(v_scale, "v_scale", torch.float32)
    _dev(block_tables, "block_tables", torch.int32), _dev(ctx_lens, "ctx_lens", torch.int32)
    nb, hkv, bs, d = k_pool.shape
    check_attention_shapes(q.shape, k_pool.shape, block_tables.shape, ctx_lens.shape)
    B, hq, _ = q.shape
    mbs = block_tables.shape[1]
    if max_context is None:
        max_context = mbs * bs
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if out is None:
        out = torch.empty_like(q)
    need = workspace_bytes(B, hq, d, max_context, partition_size)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_len = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(lib().rkv_decode_attention_q(out.data_ptr(), q.data_ptr(), k_pool.data_ptr(),
                                       v_pool.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
                                       block_tables.data_ptr(), mbs, ctx_lens.data_ptr(), B, hq,
                                       hkv, d, bs, nb, max_context, float(scale), _qcode(fmt),
                                       partition_size, ws_ptr, ws_len, _stream(q)))
    return out


def prefill_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                      block_tables: torch.Tensor, q_start: torch.Tensor, ctx_lens: torch.Tensor,
                      scale: float | None = None, *, max_q_len: int | None = None,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """Causal prefill attention: q [total, Hq, D] fp32 -> out [total, Hq, D].

    Sequence b owns rows q_start[b] .. q_start[b+1]-1 (int32 [B+1]); its new
    tokens are the last ones of its ctx_lens[b] cached tokens (appended
    beforehand).  max_q_len bounds every sequence's new-token count (computed
    from q_start, with a device sync, when not given).
    """
    _dev(q, "q", torch.float32), _dev(k_pool, "k_pool"), _dev(v_pool, "v_pool")
    _dev(block_tables, "block_tables", torch.int32), _dev(ctx_lens, "ctx_lens", torch.int32)
    _dev(q_start, "q_start", torch.int32)
    nb, hkv, bs, d = k_pool.shape
    total, hq, dq = q.shape
    B = ctx_lens.shape[0]
    check_attention_shapes(q.shape, k_pool.shape, block_tables.shape, ctx_lens.shape,
                           q_start.shape)
    if max_q_len is None:
        max_q_len = int((q_start[1:] - q_start[:-1]).max().item()) if B else 0
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if out is None:
        out = torch.zeros_like(q)
    check(lib().rkv_prefill_attention(out.data_ptr(), q.data_ptr(), k_pool.data_ptr(),
                                      v_pool.data_ptr(), block_tables.data_ptr(),
                                      block_tables.shape[1], q_start.data_ptr(),
                                      ctx_lens.data_ptr(), B, hq, hkv, d, bs, nb, max_q_len,
                                      float(scale), _dtype_code(k_pool), _stream(q)))
    return out


class DeviceBlockManager:
    """The FIFO paged block manager with its state in device memory
    (``rkv_dbm_*``): same ids in the same tables as the host ``PagedCache``
    for the same calls, but every operation is enqueued on the stream, so a
    decode step (reserve, slot mapping, append, attention) needs no host
    round trip.  Sequences are addressed by slot (0 .. max_seqs-1)."""

    def __init__(self, num_blocks: int, block_size: int = 16, max_seqs: int = 256,
                 max_blocks_per_seq: int = 256, device=None):
        self.device = torch.device(device if device is not None else "cuda")
        self.num_blocks, self.block_size = num_blocks, block_size
        self.max_seqs, self.max_blocks = max_seqs, max_blocks_per_seq
        s = torch.cuda.current_stream(self.device).cuda_stream
        self._h = lib().rkv_dbm_create(num_blocks, block_size, max_seqs, max_blocks_per_seq, s)
        if not self._h:
            raise _lib.RkvError(-1, lib().rkv_last_error().decode())

    def close(self) -> None:
        """Frees the device state (hipFree waits for the work in flight)."""
        if getattr(self, "_h", None):
            lib().rkv_dbm_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown
            pass

    def _s(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def _i32(self, x) -> torch.Tensor:
        return torch.as_tensor(x, dtype=torch.int32, device=self.device).contiguous()

    def reserve(self, slots, num_tokens) -> None:
        """Grow each slot's table to ceil(num_tokens / block_size) blocks
        (all or nothing; failures show in ``status()``)."""
        sl, nt = self._i32(slots), self._i32(num_tokens)
        assert sl.numel() == nt.numel()
        check(lib().rkv_dbm_reserve(self._h, sl.data_ptr(), nt.data_ptr(), sl.numel(), self._s()))

    def free(self, slots) -> None:
        sl = self._i32(slots)
        check(lib().rkv_dbm_free(self._h, sl.data_ptr(), sl.numel(), self._s()))

    def slot_mapping(self, slots, positions) -> torch.Tensor:
        sl, pos = self._i32(slots), self._i32(positions)
        out = torch.empty(sl.numel(), dtype=torch.int64, device=self.device)
        check(lib().rkv_dbm_slot_mapping(self._h, sl.data_ptr(), pos.data_ptr(), sl.numel(),
                                         out.data_ptr(), self._s()))
        return out

    def batch_tables(self, slots, max_blocks: int) -> torch.Tensor:
        sl = self._i32(slots)
        out = torch.empty((sl.numel(), max_blocks), dtype=torch.int32, device=self.device)
        check(lib().rkv_dbm_batch_tables(self._h, sl.data_ptr(), sl.numel(), out.data_ptr(),
                                         max_blocks, self._s()))
        return out

    def status(self, clear: bool = False):
        """(free blocks, error bits); synchronises the stream."""
        import ctypes as C
        nf, err = C.c_int64(0), C.c_int32(0)
        check(lib().rkv_dbm_status(self._h, C.addressof(nf), C.addressof(err), int(clear),
                                   self._s()))
        return nf.value, err.value

    def download(self):
        """(tables [max_seqs, max_blocks], lengths [max_seqs], free list front
        first) as numpy arrays; synchronises the stream."""
        import ctypes as C
        import numpy as np
        tables = np.empty((self.max_seqs, self.max_blocks), np.int32)
        lengths = np.empty(self.max_seqs, np.int32)
        free = np.empty(self.num_blocks, np.int32)
        nf = C.c_int64(0)
        check(lib().rkv_dbm_download(self._h, tables.ctypes.data, lengths.ctypes.data,
                                     free.ctypes.data, C.addressof(nf), self._s()))
        return tables, lengths, free[:nf.value].copy()


__all__ = ["append", "gather", "copy_blocks", "decode_attention", "prefill_attention",
           "append_q", "gather_q", "decode_attention_q", "workspace_bytes",
           "DeviceBlockManager", "_lib", "partition_size_for", "decode_attention_append",
           "decode_attention_append_q"]
