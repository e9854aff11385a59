"""CPU checks of the C ABI: the library loads, exports every declared symbol,
and rejects bad arguments on the host before any launch (no GPU needed)."""
import ctypes as C
import os
import re

import pytest

from rustral_amd import _lib
from rustral_amd._lib import (RKV_BF16, RKV_ERR_INVALID_ARG, RKV_ERR_UNSUPPORTED,
                              RKV_ERR_WORKSPACE, RKV_F32, RKV_FP8, RKV_I8)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    inc = os.path.join(ROOT, "include")
    for f in os.listdir(inc):
        if f.endswith(".h"):
            text = open(os.path.join(inc, f)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(rkv_\w+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_symbols()
    assert len(names) >= 10
    for n in sorted(names):
        assert hasattr(L, n), f"{n} declared in include/ but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert L.rkv_version() >= 100


def _decode(**kw):
    a = dict(out=16, q=16, k=16, v=16, bt=16, mbs=4, cl=16, B=2, hq=8, hkv=2, d=128, bs=16,
             nb=10, maxc=64, scale=0.1, dt=RKV_BF16, ps=0, ws=None, wsb=0, s=None)
    a.update(kw)
    return _lib.lib().rkv_decode_attention(a["out"], a["q"], a["k"], a["v"], a["bt"], a["mbs"],
                                           a["cl"], a["B"], a["hq"], a["hkv"], a["d"], a["bs"],
                                           a["nb"], a["maxc"], a["scale"], a["dt"], a["ps"],
                                           a["ws"], a["wsb"], a["s"])


@pytest.mark.parametrize("kw,code", [
    (dict(d=48), RKV_ERR_UNSUPPORTED),
    (dict(bs=32), RKV_ERR_UNSUPPORTED),
    (dict(hq=6, hkv=2), RKV_ERR_UNSUPPORTED),     # G = 3
    (dict(hq=7, hkv=2), RKV_ERR_INVALID_ARG),     # not a multiple
    (dict(dt=5), RKV_ERR_INVALID_ARG),
    (dict(q=None), RKV_ERR_INVALID_ARG),
    (dict(out=8), RKV_ERR_INVALID_ARG),           # misaligned
    (dict(maxc=1000, mbs=100), RKV_ERR_WORKSPACE),  # needs split-K partials
    (dict(ps=100), RKV_ERR_UNSUPPORTED),            # not a multiple of 64 tokens
    (dict(ps=704), RKV_ERR_UNSUPPORTED),            # above the largest build
])
def test_decode_rejects_bad_arguments(kw, code):
    assert _decode(**kw) == code
    assert _lib.lib().rkv_last_error().decode()


def test_decode_zero_sequences_is_a_no_op():
    assert _decode(B=0, out=None, q=None) == 0
    assert _lib.lib().rkv_last_error().decode() == ""


def test_workspace_size():
    L = _lib.lib()
    P = L.rkv_decode_partition_size(0, 128, RKV_BF16, 4096)
    assert P == 640
    # the default workspace (partition size 0) is sized for the smallest size
    # a call picks by itself, 512
    assert L.rkv_decode_workspace_bytes(64, 32, 128, 512, 0) == 0  # one partition
    assert L.rkv_decode_workspace_bytes(64, 32, 128, 640, 0) > 0
    ws = L.rkv_decode_workspace_bytes(64, 32, 128, 4096, 0)
    rows = 64 * 32 * -(-4096 // 512)
    assert ws >= rows * (128 + 2) * 4
    # each pool dtype has its default partition size at a max_context; the
    # default workspace (partition size 0) covers every one of them
    for maxc in (4096, 65536):
        ws = L.rkv_decode_workspace_bytes(8, 32, 128, maxc, 0)
        for dt in (RKV_F32, RKV_BF16, RKV_I8, RKV_FP8):
            Pd = L.rkv_decode_partition_size(0, 128, dt, maxc)
            assert Pd > 0 and Pd % 64 == 0
            assert ws >= L.rkv_decode_workspace_bytes(8, 32, 128, maxc, Pd)
    # the split entry points' default is 640 for every dtype and context
    for dt in (RKV_F32, RKV_BF16, RKV_I8, RKV_FP8):
        for maxc in (16, 4096, 65536):
            assert L.rkv_decode_partition_size(0, 128, dt, maxc) == 640
    # the one-call pick by shape: bf16, head_dim 128, <= 4 query heads per KV
    # head; 1280 with work for >= 1200 such partitions, 768 with work for >=
    # 1000 of those, 640 with work for >= 800 partitions of 512, else 512
    # (configs[2]: 768; configs[3] and 256 x 8192: 1280; configs[2]'s share
    # of one GPU of 8: 512; above the 512 tier, 8 heads per KV head, head_dim
    # 64, fp32 and 1-byte pools: 640)
    F = L.rkv_decode_partition_size_for
    assert F(0, 64, 32, 8, 128, RKV_BF16, 4096) == 768
    assert F(0, 8, 32, 8, 128, RKV_BF16, 65536) == 1280
    assert F(0, 256, 32, 8, 128, RKV_BF16, 8192) == 1280
    assert F(0, 8, 32, 8, 128, RKV_BF16, 4096) == 512     # 8 sequences (a DP share)
    assert F(0, 64, 4, 1, 128, RKV_BF16, 4096) == 512     # one KV head (a TP share)
    assert F(0, 8, 64, 8, 128, RKV_BF16, 4096) == 512     # small calls: every shape
    assert F(0, 8, 32, 8, 64, RKV_BF16, 4096) == 512
    assert F(0, 8, 32, 8, 128, RKV_F32, 4096) == 512
    for dt in (RKV_I8, RKV_FP8):  # 1-byte pools: 512 up to twice the work
        assert F(0, 8, 32, 8, 128, dt, 4096) == 512
        assert F(0, 32, 32, 8, 128, dt, 4096) == 512
        assert F(0, 64, 32, 8, 128, dt, 4096) == 640
        assert F(0, 1, 32, 8, 128, dt, 204800) == 640     # 8 * 102400 = 1600 x 512
        assert F(0, 1, 32, 8, 128, dt, 204799) == 512
    assert F(0, 4, 32, 8, 128, RKV_BF16, 32768) == 640
    assert F(0, 64, 64, 8, 128, RKV_BF16, 4096) == 640    # G = 8
    assert F(0, 64, 32, 8, 64, RKV_BF16, 4096) == 640     # head_dim 64
    assert F(0, 64, 8, 8, 128, RKV_BF16, 4096) == 768     # G = 1
    for dt in (RKV_F32, RKV_I8, RKV_FP8):
        assert F(0, 256, 32, 8, 128, dt, 65536) == 640
    # a request is the request, with the rules of rkv_decode_partition_size
    assert F(512, 64, 32, 8, 128, RKV_BF16, 4096) == 512
    assert F(1024, 64, 32, 8, 128, RKV_BF16, 4096) == 1024
    assert F(1024, 64, 32, 8, 128, RKV_F32, 4096) == RKV_ERR_UNSUPPORTED
    # the thresholds: 1200 x 1280 and 1000 x 768 KV-head tokens (contexts
    # taken as uniform up to max_context)
    assert F(0, 1, 32, 8, 128, RKV_BF16, 384000) == 1280  # 8 * 192000 = 1.536M
    assert F(0, 1, 32, 8, 128, RKV_BF16, 383999) == 768
    assert F(0, 1, 32, 8, 128, RKV_BF16, 192000) == 768   # 8 * 96000 = 768k
    assert F(0, 1, 32, 8, 128, RKV_BF16, 191999) == 640
    assert F(0, 1, 32, 8, 128, RKV_BF16, 102400) == 640   # 8 * 51200 = 800 x 512
    assert F(0, 1, 32, 8, 128, RKV_BF16, 102399) == 512
    # the default workspace covers the smallest pick
    for maxc in (4096, 65536):
        assert (L.rkv_decode_workspace_bytes(8, 32, 128, maxc, 0)
                >= L.rkv_decode_workspace_bytes(8, 32, 128, maxc, 512))
    # bf16 pools also take multiples of 128 up to 1280; the others do not
    for req in (768, 896, 1024, 1280):
        assert L.rkv_decode_partition_size(req, 128, RKV_BF16, 4096) == req
        for dt in (RKV_F32, RKV_I8, RKV_FP8):
            assert L.rkv_decode_partition_size(req, 128, dt, 4096) == RKV_ERR_UNSUPPORTED
    for req in (704, 832, 1408):
        assert L.rkv_decode_partition_size(req, 128, RKV_BF16, 4096) == RKV_ERR_UNSUPPORTED
    # a request is honoured when it is a multiple of 64 up to 640
    for req in (64, 128, 320, 512, 576, 640):
        assert L.rkv_decode_partition_size(req, 128, RKV_BF16, 4096) == req
    for req in (100, 704, 1400):
        assert L.rkv_decode_partition_size(req, 128, RKV_BF16, 4096) == RKV_ERR_UNSUPPORTED
    for req in (100, 704, 1024):
        assert L.rkv_decode_partition_size(req, 128, RKV_F32, 4096) == RKV_ERR_UNSUPPORTED


def test_copy_kernels_reject_bad_arguments():
    L = _lib.lib()
    assert L.rkv_append(16, 16, 0, 16, 16, 0, 1024, 128, 16, 4, 1, 8, 12, 16, 10, RKV_F32,
                        None) == RKV_ERR_UNSUPPORTED  # head_dim 12
    assert L.rkv_append(16, 16, 0, 16, 16, 0, 1022, 128, 16, 4, 1, 8, 128, 16, 10, RKV_F32,
                        None) == RKV_ERR_INVALID_ARG  # stride not a multiple of 4
    assert L.rkv_append(16, 16, 0, 16, 16, 0, 1024, 128, 16, 0, 1, 8, 128, 16, 10, RKV_F32,
                        None) == 0  # nothing to do
    assert L.rkv_gather(16, 16, 16, 16, 16, 4, 16, None, 2, 8, 128, 16, 10, 64, RKV_F32, RKV_BF16,
                        None) == RKV_ERR_INVALID_ARG  # f32 -> bf16 not offered
    assert L.rkv_copy_blocks(16, 16, 0, 1, 16, 3, 100, 10, None) == RKV_ERR_INVALID_ARG
    assert L.rkv_copy_blocks(16, 16, 0, 1, 16, 0, 4096, 10, None) == 0


def test_prefill_rejects_bad_arguments():
    """Argument checks of rkv_prefill_attention run before any launch."""
    L = _lib.lib()

    def call(hq=8, hkv=2, d=128, bs=16, dt=RKV_BF16, B=2, mq=16, mbs=4):
        return L.rkv_prefill_attention(16, 16, 16, 16, 16, mbs, 16, 16, B, hq, hkv, d, bs, 10, mq,
                                       0.1, dt, None)
    assert call(bs=8) == RKV_ERR_UNSUPPORTED
    assert call(d=48) == RKV_ERR_UNSUPPORTED
    assert call(hq=6, hkv=2) == RKV_ERR_UNSUPPORTED
    assert call(hq=7, hkv=2) == RKV_ERR_INVALID_ARG
    assert call(dt=7) == RKV_ERR_INVALID_ARG
    assert call(B=-1) == RKV_ERR_INVALID_ARG
    assert call(B=0) == 0 and call(mq=0) == 0          # nothing to do: no launch
    assert L.rkv_prefill_attention(None, 16, 16, 16, 16, 4, 16, 16, 2, 8, 2, 128, 16, 10, 16,
                                   0.1, RKV_BF16, None) == RKV_ERR_INVALID_ARG


def test_recipe_ops_reject_bad_arguments():
    """rkv_softmax_dim / rkv_matmul / rkv_transpose / rkv_mul_scalar check
    sizes and pointers before any launch; empty shapes are no-ops."""
    L = _lib.lib()
    assert L.rkv_softmax_dim(16, 16, 2, 0, 1, None) == RKV_ERR_INVALID_ARG  # axis size 0
    assert "axis" in L.rkv_last_error().decode()
    assert L.rkv_softmax_dim(16, 16, -1, 4, 1, None) == RKV_ERR_INVALID_ARG
    assert L.rkv_softmax_dim(None, 16, 2, 4, 1, None) == RKV_ERR_INVALID_ARG
    assert L.rkv_softmax_dim(16, 16, 1 << 40, 1 << 20, 1 << 10, None) == RKV_ERR_INVALID_ARG
    assert L.rkv_softmax_dim(None, None, 0, 4, 1, None) == 0
    assert L.rkv_matmul(16, 16, 16, -1, 2, 2, None) == RKV_ERR_INVALID_ARG
    assert L.rkv_matmul(16, None, 16, 2, 2, 2, None) == RKV_ERR_INVALID_ARG
    assert L.rkv_matmul(None, None, None, 0, 5, 3, None) == 0
    assert L.rkv_transpose(16, 16, 4, 4, None) == RKV_ERR_INVALID_ARG  # aliasing
    assert L.rkv_transpose(16, 32, -4, 4, None) == RKV_ERR_INVALID_ARG
    assert L.rkv_mul_scalar(16, 16, 2.0, -1, None) == RKV_ERR_INVALID_ARG
    assert L.rkv_mul_scalar(None, None, 2.0, 0, None) == 0


def test_attention_shape_check_rejects_mismatches_before_a_launch():
    """The host wrappers' shape check (the Rust crate's check_attention_shapes
    states the same rules): the pool's head_dim, Hq a multiple of Hkv, one
    table row and one length per sequence, B + 1 prefill offsets."""
    from rustral_amd.kv import check_attention_shapes as chk
    pool = (64, 8, 16, 128)
    chk((4, 32, 128), pool, (4, 16), (4,))
    chk((300, 32, 128), pool, (4, 16), (4,), (5,))
    for q, t, n, qs in [((4, 32, 256), (4, 16), (4,), None),   # wider rows than the pool's
                        ((4, 32, 64), (4, 16), (4,), None),
                        ((4, 12, 128), (4, 16), (4,), None),   # Hq not a multiple of Hkv
                        ((4, 32, 128), (3, 16), (4,), None),   # short tables
                        ((4, 32, 128), (4, 16), (3,), None),   # short lengths
                        ((5, 32, 128), (4, 16), (4,), None),
                        ((300, 32, 128), (4, 16), (4,), (4,)),
                        ((4, 32), (4, 16), (4,), None)]:
        with pytest.raises(ValueError):
            chk(q, pool, t, n, qs)


def test_linear_rejects_rows_too_wide_for_staging():
    L = _lib.lib()
    assert L.rkv_linear(16, 16, 16, None, 1, 8193, 4, None) == RKV_ERR_UNSUPPORTED
    assert "in_dim" in L.rkv_last_error().decode()


def test_noalloc_decode_refuses_partials_above_its_scratch():
    """rkv_decode_attention_noalloc checks the size on the host, before any
    HIP call: partials above its fixed scratch are RKV_ERR_WORKSPACE."""
    L = _lib.lib()
    cap = L.rkv_decode_noalloc_max_bytes()
    assert cap == 16 << 20
    assert L.rkv_decode_workspace_bytes(4096, 32, 128, 4096, 0) > cap
    rc = L.rkv_decode_attention_noalloc(16, 16, 16, 16, 16, 256, 16, 4096, 32, 8, 128, 16, 10,
                                        4096, 0.1, RKV_BF16, 0, None)
    assert rc == RKV_ERR_WORKSPACE and b"16 MiB" in L.rkv_last_error()


def _decode_append(**kw):
    a = dict(out=16, q=16, k=16, v=16, kn=16, vn=16, bt=16, mbs=4, cl=16, B=2, hq=8, hkv=2,
             d=128, bs=16, nb=10, maxc=64, scale=0.1, dt=RKV_BF16, ps=0, ws=None, wsb=0, s=None)
    a.update(kw)
    return _lib.lib().rkv_decode_attention_append(
        a["out"], a["q"], a["k"], a["v"], a["kn"], a["vn"], a["bt"], a["mbs"], a["cl"], a["B"],
        a["hq"], a["hkv"], a["d"], a["bs"], a["nb"], a["maxc"], a["scale"], a["dt"], a["ps"],
        a["ws"], a["wsb"], a["s"])


@pytest.mark.parametrize("kw,code", [
    (dict(dt=RKV_F32), RKV_ERR_UNSUPPORTED),     # fused append: bf16 pools only
    (dict(dt=RKV_I8), RKV_ERR_UNSUPPORTED),
    (dict(kn=None), RKV_ERR_INVALID_ARG),
    (dict(vn=8), RKV_ERR_INVALID_ARG),           # misaligned
    (dict(d=48), RKV_ERR_UNSUPPORTED),
    (dict(maxc=1000, mbs=100), RKV_ERR_WORKSPACE),
    (dict(ps=100), RKV_ERR_UNSUPPORTED),
])
def test_decode_append_rejects_bad_arguments(kw, code):
    assert _decode_append(**kw) == code
    assert _lib.lib().rkv_last_error().decode()


def test_decode_append_zero_sequences_is_a_no_op():
    assert _decode_append(B=0, kn=None, vn=None, out=None, q=None) == 0


def test_decode_append_q_rejects_bad_arguments():
    L = _lib.lib()

    def call(dt=RKV_I8, kn=16, vn=16, d=128):
        return L.rkv_decode_attention_append_q(16, 16, 16, 16, 16, 16, kn, vn, 16, 4, 16, 2, 8,
                                               2, d, 16, 10, 64, 0.1, dt, 0, None, 0, None)
    assert call(dt=RKV_BF16) == RKV_ERR_INVALID_ARG
    assert call(kn=None) == RKV_ERR_INVALID_ARG
    assert call(vn=8) == RKV_ERR_INVALID_ARG
    assert call(d=32) == RKV_ERR_UNSUPPORTED
    assert call(dt=RKV_FP8, d=48) == RKV_ERR_UNSUPPORTED
