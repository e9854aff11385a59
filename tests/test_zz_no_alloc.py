"""rkv_decode_attention_noalloc (the entry point that allocates nothing) on the
GPU: called through the C ABI, its output equals rkv_decode_attention's with a
caller workspace, bit for bit (the same kernels on the same inputs), on two
calls in a row -- the second one smaller, so it runs over the scratch the
first call left behind -- and it matches the oracle to the decode tolerance.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from rustral_amd import _lib, kv
from rustral_amd._lib import RKV_BF16, RKV_ERR_WORKSPACE, RKV_F32
from tests.gpu_util import say, to_dev, to_np
from tests.helpers import assert_allclose_ref, make_pool, make_tables

pytestmark = pytest.mark.gpu


def _case(seed, ctx, hq, hkv, d, dtype):
    rng = np.random.default_rng(seed)
    nb = int(sum((int(c) + 15) // 16 for c in ctx)) + 2
    kp, vp, _, _ = make_pool(rng, nb, hkv, 16, d, dtype)
    tables = make_tables(rng, ctx, 16, nb)
    q = rng.standard_normal((len(ctx), hq, d)).astype(np.float32)
    return q, kp, vp, tables


def _noalloc(dev, q, kp, vp, tables, ctx, scale, dtype_code):
    B, hq, d = q.shape
    nb, hkv, bs, _ = kp.shape
    gq, gk, gv = to_dev(q, dev), to_dev(kp, dev), to_dev(vp, dev)
    gt, gc = to_dev(tables, dev), to_dev(ctx, dev)
    out = torch.full_like(gq, float("nan"))
    s = torch.cuda.current_stream(dev).cuda_stream
    rc = _lib.lib().rkv_decode_attention_noalloc(
        out.data_ptr(), gq.data_ptr(), gk.data_ptr(), gv.data_ptr(), gt.data_ptr(),
        tables.shape[1], gc.data_ptr(), B, hq, hkv, d, bs, nb, tables.shape[1] * bs,
        float(scale), dtype_code, 0, s)
    _lib.check(rc)
    ref = kv.decode_attention(gq, gk, gv, gt, gc, scale)   # caller-owned workspace
    torch.cuda.synchronize()
    return to_np(out), to_np(ref)


@pytest.mark.parametrize("dtype,code", [("bf16", RKV_BF16), ("f32", RKV_F32)])
def test_noalloc_equals_workspace_entry_point_twice(dev, dtype, code):
    d, hq, hkv = 128, 32, 8
    scale = float(np.float32(1.0 / math.sqrt(d)))
    cases = [
        np.array([3000, 17, 1290, 640, 641, 2500, 1, 4096], np.int32),   # many partitions
        np.array([700, 5, 1300], np.int32),                               # smaller second call
    ]
    for i, ctx in enumerate(cases):
        say(f"noalloc dtype={dtype} call={i} B={len(ctx)} max_ctx={ctx.max()}")
        q, kp, vp, tables = _case(50 + i, ctx, hq, hkv, d, dtype)
        got, ref = _noalloc(dev, q, kp, vp, tables, ctx, scale, code)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"call {i}"
        want = oracle.decode_attention(q, kp, vp, tables, ctx, scale)
        assert_allclose_ref(got, want, 1e-3, 1e-4, f"noalloc call {i} vs oracle")


def test_noalloc_rejects_partials_above_the_scratch(dev):
    # B 4096 x 32 heads x 7 partitions of partials is well above 16 MiB;
    # refused on the host before any launch
    L = _lib.lib()
    need = L.rkv_decode_workspace_bytes(4096, 32, 128, 4096, 0)
    assert need > L.rkv_decode_noalloc_max_bytes()
    rc = L.rkv_decode_attention_noalloc(16, 16, 16, 16, 16, 256, 16, 4096, 32, 8, 128, 16, 10,
                                        4096, 0.1, RKV_BF16, 0, None)
    assert rc == RKV_ERR_WORKSPACE
    assert b"16 MiB" in L.rkv_last_error()
