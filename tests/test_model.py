"""Model glue around the path (benchmark configs[0]): generator, oracle pins,
device ops and the end-to-end greedy decoder.

CPU tests pin the oracle's decoder glue (oracle/rkv_oracle.c) against an
independent float64 numpy formulation and against closed forms, and pin the
product's generator against numpy's PCG64.  GPU tests compare every device
op with the oracle (bit-exact where the summation order is the reference's;
gelu within a few ulps because tanh comes from the device library) and run
configs[0] end to end: the 64 generated tokens must equal the oracle's.
"""
import math

import numpy as np
import pytest

import oracle
from rustral_amd import model

PCG_INC = (0xDA3E39CB94B95BDB << 1) | 1


# ---- generator -------------------------------------------------------------------

@pytest.mark.parametrize("seed", [0, 1, 12345, 2 ** 63 + 7])
def test_rng_matches_numpy_pcg64(seed):
    bg = np.random.PCG64()
    st = bg.state
    st["state"] = {"state": seed, "inc": PCG_INC}
    st["has_uint32"], st["uinteger"] = 0, 0
    bg.state = st
    np.testing.assert_array_equal(model.rng_raw(seed, 1000), bg.random_raw(1000))


def test_fill_normal_is_box_muller_of_the_stream():
    raw = model.rng_raw(7, 2000).astype(np.uint64)
    u = (raw >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(1.0 - u1))
    z = np.empty(2000)
    z[0::2], z[1::2] = r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)
    want = (0.02 * z).astype(np.float32)
    got = model.fill_normal(2000, 7, 0.02)
    ulps = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1, "fp32 results differ by more than 1 ulp (libm vs numpy in double)"


def test_fill_normal_statistics():
    from scipy import stats
    z = model.fill_normal(400_001, 3, 1.0).astype(np.float64)
    assert abs(z.mean()) < 0.005 and abs(z.std() - 1.0) < 0.005
    assert stats.kstest(z, "norm").pvalue > 1e-3
    assert np.array_equal(z, model.fill_normal(400_001, 3, 1.0))
    assert not np.array_equal(z[:100], model.fill_normal(100, 4, 1.0))


def test_param_layout_and_init():
    cfg = model.config()
    ocfg = oracle.decoder_config()
    n = model.param_count(cfg)
    assert n == oracle.decoder_param_count(ocfg) == 652_800
    for kw in [dict(n_kv_heads=2), dict(n_layers=3, d_ff=256), dict(vocab=17, d_model=64, n_heads=2, n_kv_heads=1)]:
        assert model.param_count(model.config(**kw)) == oracle.decoder_param_count(
            oracle.decoder_config(**kw))
    p = model.init_params(cfg, seed=0)
    V, d, f = 1000, 128, 512
    np.testing.assert_array_equal(p[:V * d], model.fill_normal(V * d, 0, 0.02))
    off = V * d
    per = 2 * d + 4 * (d * d + d) + 2 * d + (f * d + f) + (d * f + d)
    for l in range(2):
        o = off + l * per
        assert (p[o:o + d] == 1).all() and (p[o + d:o + 2 * d] == 0).all()       # ln1
        bq = o + 2 * d + d * d
        assert (p[bq:bq + d] == 0).all()
        ln2 = o + 2 * d + 4 * (d * d + d)
        assert (p[ln2:ln2 + d] == 1).all() and (p[ln2 + d:ln2 + 2 * d] == 0).all()
    fin = off + 2 * per
    assert (p[fin:fin + d] == 1).all() and (p[fin + d:fin + 2 * d] == 0).all()
    assert abs(p[fin + 2 * d:].std() - 0.02) < 0.001
    assert np.array_equal(p, model.init_params(cfg, seed=0))


# ---- oracle glue pins ------------------------------------------------------------

def test_oracle_linear_known_answers():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 16)).astype(np.float32)
    b = rng.standard_normal(16).astype(np.float32)
    # identity weight: y = x + b exactly
    np.testing.assert_array_equal(oracle.linear(x, np.eye(16, dtype=np.float32), b), x + b)
    w = rng.standard_normal((7, 16)).astype(np.float32)
    ref = x.astype(np.float64) @ w.T.astype(np.float64)
    np.testing.assert_allclose(oracle.linear(x, w), ref, rtol=1e-5, atol=1e-5)
    # serial order: a sum that cancels only when added left to right
    x1 = np.array([[1e8, 1.0, -1e8]], np.float32)
    w1 = np.ones((1, 3), np.float32)
    assert oracle.linear(x1, w1)[0, 0] == 0.0          # (1e8 + 1) - 1e8 in fp32


def test_oracle_layer_norm_pins():
    rng = np.random.default_rng(2)
    g = rng.standard_normal(64).astype(np.float32)
    b = rng.standard_normal(64).astype(np.float32)
    const = np.full((1, 64), 3.5, np.float32)
    np.testing.assert_array_equal(oracle.layer_norm(const, g, b), b[None])   # x - mean = 0
    x = rng.standard_normal((5, 64)).astype(np.float32) * 3 + 1
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    var = ((xd - mu) ** 2).mean(1, keepdims=True)
    ref = (xd - mu) / np.sqrt(var + 1e-5) * g + b
    np.testing.assert_allclose(oracle.layer_norm(x, g, b), ref, rtol=1e-5, atol=1e-5)


def test_oracle_gelu_and_pe_pins():
    x = np.linspace(-8, 8, 1001).astype(np.float32)
    xd = x.astype(np.float64)
    ref = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)))
    np.testing.assert_allclose(oracle.gelu(x), ref, rtol=1e-5, atol=1e-6)
    assert oracle.gelu(np.zeros(1, np.float32))[0] == 0.0
    pe = oracle.positional_encoding(96, 128)
    np.testing.assert_array_equal(pe[0, 0::2], 0.0)    # sin 0
    np.testing.assert_array_equal(pe[0, 1::2], 1.0)    # cos 0
    pos = np.arange(96)[:, None].astype(np.float64)
    i = np.arange(128)[None]
    ang = pos / 10000.0 ** ((2 * (i // 2)) / 128.0)
    ref = np.where(i % 2 == 0, np.sin(ang), np.cos(ang))
    np.testing.assert_allclose(pe, ref, atol=5e-5)   # fp32 angle rounding at large pos


def _np_decoder_logits(params, cfg, ids):
    """Independent float64 formulation: the whole sequence at once with a
    causal mask (not the oracle's per-token cache loop)."""
    d, V, f, H, Hk, L = cfg["d_model"], cfg["vocab"], cfg["d_ff"], cfg["n_heads"], \
        cfg["n_kv_heads"], cfg["n_layers"]
    dh = d // H
    kvd = Hk * dh
    P = params.astype(np.float64)
    o = 0

    def take(*shape):
        nonlocal o
        n = int(np.prod(shape))
        a = P[o:o + n].reshape(shape)
        o += n
        return a

    def ln(x, g, b):
        mu = x.mean(-1, keepdims=True)
        return (x - mu) / np.sqrt(((x - mu) ** 2).mean(-1, keepdims=True) + cfg["eps"]) * g + b

    T = len(ids)
    E = take(V, d)
    pe = oracle.positional_encoding(T, d).astype(np.float64)
    x = E[ids] + pe
    for _ in range(L):
        g1, b1 = take(d), take(d)
        wq, bq, wk, bk, wv, bv = take(d, d), take(d), take(kvd, d), take(kvd), take(kvd, d), take(kvd)
        wo, bo = take(d, d), take(d)
        g2, b2 = take(d), take(d)
        w1, c1, w2, c2 = take(f, d), take(f), take(d, f), take(d)
        h = ln(x, g1, b1)
        q = (h @ wq.T + bq).reshape(T, H, dh)
        k = (h @ wk.T + bk).reshape(T, Hk, dh)
        v = (h @ wv.T + bv).reshape(T, Hk, dh)
        out = np.empty((T, H, dh))
        mask = np.triu(np.full((T, T), -np.inf), 1)
        for hh in range(H):
            kh = hh // (H // Hk)
            s = q[:, hh] @ k[:, kh].T / math.sqrt(dh) + mask
            s = np.exp(s - s.max(1, keepdims=True))
            out[:, hh] = (s / s.sum(1, keepdims=True)) @ v[:, kh]
        x = x + out.reshape(T, d) @ wo.T + bo
        h = ln(x, g2, b2)
        u = h @ w1.T + c1
        u = 0.5 * u * (1 + np.tanh(math.sqrt(2 / math.pi) * (u + 0.044715 * u ** 3)))
        x = x + u @ w2.T + c2
    gf, bf = take(d), take(d)
    wlm = take(V, d)
    assert o == P.size
    return ln(x, gf, bf) @ wlm.T


@pytest.mark.parametrize("kw", [dict(), dict(n_kv_heads=2, n_layers=1, vocab=300)])
def test_oracle_decoder_matches_independent_float64_model(kw):
    cfg = dict(oracle.CONFIG0, **kw)
    ocfg = oracle.decoder_config(**kw)
    rng = np.random.default_rng(5)
    params = (rng.standard_normal(oracle.decoder_param_count(ocfg)) * 0.05).astype(np.float32)
    prompt = rng.integers(0, cfg["vocab"], 12).astype(np.int32)
    toks, lg = oracle.decoder_generate(ocfg, params, prompt, 20, logits=True)
    seq = np.concatenate([prompt, toks[:-1]])
    ref = _np_decoder_logits(params, cfg, seq)[len(prompt) - 1:]
    np.testing.assert_allclose(lg, ref, atol=2e-5, rtol=1e-4)
    for t in range(20):
        top2 = np.sort(ref[t])[-2:]
        if top2[1] - top2[0] > 1e-4:                   # no near-tie: the choice is fixed
            assert toks[t] == int(np.argmax(ref[t]))


# ---- device ops and the decoder (GPU) ----------------------------------------------

@pytest.fixture
def torch_dev(dev):
    import torch
    return torch, dev


@pytest.mark.gpu
@pytest.mark.parametrize("rows,i,o", [(1, 128, 128), (1, 128, 512), (1, 512, 128), (3, 128, 1000),
                                      (5, 33, 7), (2, 8192, 70), (1, 4097, 65)])
def test_gpu_linear_bit_exact(torch_dev, rows, i, o):
    torch, dev = torch_dev
    rng = np.random.default_rng(rows * 100 + i + o)
    x = rng.standard_normal((rows, i)).astype(np.float32)
    w = (rng.standard_normal((o, i)) * 0.05).astype(np.float32)
    b = rng.standard_normal(o).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    got = model.linear(t(x), t(w), t(b)).cpu().numpy()
    assert np.array_equal(got, oracle.linear(x, w, b))
    got = model.linear(t(x), t(w)).cpu().numpy()
    assert np.array_equal(got, oracle.linear(x, w))


@pytest.mark.gpu
def test_gpu_layer_norm_add_embed_bit_exact(torch_dev):
    torch, dev = torch_dev
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((4, 128)) * 2 + 0.5).astype(np.float32)
    g = rng.standard_normal(128).astype(np.float32)
    b = rng.standard_normal(128).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    assert np.array_equal(model.layer_norm(t(x), t(g), t(b)).cpu().numpy(),
                          oracle.layer_norm(x, g, b))
    y = rng.standard_normal((4, 128)).astype(np.float32)
    assert np.array_equal(model.add(t(x), t(y)).cpu().numpy(), x + y)
    table = rng.standard_normal((50, 128)).astype(np.float32)
    pe = oracle.positional_encoding(20, 128)
    ids = np.array([3, 49, 0, 7], np.int32)
    pos = np.array([0, 5, 19, 2], np.int32)
    got = model.embed(t(table), t(ids), t(pe), t(pos)).cpu().numpy()
    assert np.array_equal(got, table[ids] + pe[pos])
    bad = model.embed(t(table), t(np.array([50, -1], np.int32))).cpu().numpy()
    assert np.isnan(bad).all()


@pytest.mark.gpu
def test_gpu_decoder_on_a_caller_stream(dev):
    """The decoder built on a caller's (non-default) stream captures and
    replays its launch sequence on that stream; tokens equal the CPU
    decoder's on the first call (capture) and on later ones (replays)."""
    import torch
    from tests.gpu_util import say
    say("decoder on a caller stream")
    cfg = model.config()
    params = model.init_params(cfg, seed=3, std=0.02)
    rng = np.random.default_rng(4)
    side = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(side):
        dec = model.Decoder(cfg, params)
        for _ in range(3):
            prompt = rng.integers(0, 1000, 12).astype(np.int32)
            got = dec.generate(prompt, 24)
            want = oracle.decoder_generate(oracle.decoder_config(), params, prompt, 24)
            assert got.tolist() == want.tolist()
    torch.cuda.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("n,d,hq,hkv,dtype,ln,bias", [
    (1, 128, 4, 4, "f32", True, True),        # configs[0] decode row
    (300, 128, 4, 2, "f32", True, True),      # a prompt's rows, GQA
    (7, 256, 8, 1, "bf16", True, False),
    (5, 4096, 32, 8, "bf16", False, True),    # Llama-3-8B layer shape
    (3, 33, 3, 1, "f32", True, True)])        # odd d_model: the scalar weight path
def test_gpu_qkv_append_bit_exact(torch_dev, n, d, hq, hkv, dtype, ln, bias):
    """The fused LN1 -> q / k / v -> append launch equals the oracle's
    layer_norm + 3 x linear + append bit for bit (pools and q), with padding
    and out-of-range slots appending nothing."""
    torch, dev = torch_dev
    rng = np.random.default_rng(n * 7 + d + hq)
    hd = d // hq
    kvd = hkv * hd
    nb, bs = (n + 15) // 16 + 3, 16
    x = (rng.standard_normal((n, d)) * 1.5 + 0.3).astype(np.float32)
    wq, wk, wv = ((rng.standard_normal((o, d)) * 0.05).astype(np.float32) for o in (hq * hd, kvd, kvd))
    bq, bk, bv = (rng.standard_normal(o).astype(np.float32) if bias else None for o in (hq * hd, kvd, kvd))
    g = rng.standard_normal(d).astype(np.float32) if ln else None
    b = rng.standard_normal(d).astype(np.float32) if ln else None
    slots = rng.permutation(nb * bs)[:n].astype(np.int64)
    slots[::5] = -1
    if n > 2:
        slots[1] = nb * bs + 3                          # outside the pool: skipped
    np_dt = np.float32
    kp = rng.standard_normal((nb, hkv, bs, hd)).astype(np_dt)
    vp = rng.standard_normal((nb, hkv, bs, hd)).astype(np_dt)
    if dtype == "bf16":
        kp, vp = oracle.bf16_from_f32(kp), oracle.bf16_from_f32(vp)
    h = oracle.layer_norm(x, g, b) if ln else x
    want_q = oracle.linear(h, wq, bq)
    k_new = oracle.linear(h, wk, bk).reshape(n, hkv, hd)
    v_new = oracle.linear(h, wv, bv).reshape(n, hkv, hd)
    want_k, want_v = kp.copy(), vp.copy()
    oracle.append(want_k, want_v, k_new, v_new, slots)
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    if dtype == "bf16":
        gk = torch.from_numpy(kp.view(np.int16)).to(dev).view(torch.bfloat16)
        gv = torch.from_numpy(vp.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        gk, gv = t(kp), t(vp)
    q = model.qkv_append(t(x), t(wq), t(wk), t(wv), gk, gv, t(slots), t(bq), t(bk), t(bv),
                         t(g), t(b))
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), want_q)
    if dtype == "bf16":
        got_k = gk.view(torch.int16).cpu().numpy().view(np.uint16)
        got_v = gv.view(torch.int16).cpu().numpy().view(np.uint16)
    else:
        got_k, got_v = gk.cpu().numpy(), gv.cpu().numpy()
    assert np.array_equal(got_k.view(np.uint8), want_k.view(np.uint8))
    assert np.array_equal(got_v.view(np.uint8), want_v.view(np.uint8))


@pytest.mark.gpu
def test_gpu_gelu_close(torch_dev):
    torch, dev = torch_dev
    x = np.linspace(-10, 10, 4097).astype(np.float32)
    got = model.gelu(torch.from_numpy(x).to(dev)).cpu().numpy()
    want = oracle.gelu(x)
    assert np.abs(got - want).max() <= 4 * np.spacing(np.abs(want).max())


@pytest.mark.gpu
def test_gpu_argmax_matches_reference_rule(torch_dev):
    torch, dev = torch_dev
    rng = np.random.default_rng(4)
    rows = [rng.standard_normal(1000).astype(np.float32) for _ in range(6)]
    rows.append(np.array([0.1, 0.5, 0.3, 0.9, 0.2] + [0.0] * 995, np.float32))  # reference fixture
    tie = rng.integers(-3, 3, 1000).astype(np.float32)
    rows.append(tie)                                                          # many equal maxima
    nan = rng.standard_normal(1000).astype(np.float32)
    nan[[10, 500]] = np.nan
    rows.append(nan)
    x = np.stack(rows)
    got = model.argmax(torch.from_numpy(x).to(dev)).cpu().numpy()
    want = [oracle.argmax(r) for r in rows]
    assert got.tolist() == want
    assert want[6] == 3 and want[7] == int(np.flatnonzero(tie == tie.max())[-1])


@pytest.mark.gpu
def test_gpu_softmax_dim_matches_oracle(torch_dev):
    """rkv_softmax_dim against the oracle's softmax_dim: the reference's golden
    rows at its tolerance (crates/core/tests/golden_microblock_ops.rs:14-26,
    rtol 1e-5 / atol 1e-6), random rows up to 4096 columns and past the
    2048-entry sum chunk, every axis of a 3-d tensor, and the NaN / -inf rules."""
    torch, dev = torch_dev
    import json
    import os
    kat = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                      "reference_kats.json")))["softmax_dim1"]
    rtol, atol = kat["tolerance"]["rtol"], kat["tolerance"]["atol"]

    def close(got, want, what):
        d = np.abs(got.astype(np.float64) - want)
        assert (d <= atol + rtol * np.abs(want)).all(), f"{what}: max abs diff {d.max()}"

    x = np.array(kat["input"], np.float32).reshape(kat["rows"], kat["cols"])
    close(model.softmax_dim(torch.from_numpy(x).to(dev), 1).cpu().numpy(),
          oracle.softmax_dim(x, 1), "golden")
    rng = np.random.default_rng(9)
    for rows, cols in [(1, 1), (3, 7), (64, 128), (5, 2048), (4, 2049), (2, 4096), (1, 70001)]:
        x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
        got = model.softmax_dim(torch.from_numpy(x).to(dev), 1).cpu().numpy()
        close(got, oracle.softmax_dim(x, 1), f"rows {rows} cols {cols}")
    x = (rng.standard_normal((6, 33, 5)) * 3).astype(np.float32)
    for dim in range(3):
        got = model.softmax_dim(torch.from_numpy(x).to(dev), dim).cpu().numpy()
        close(got, oracle.softmax_dim(x, dim), f"3-d dim {dim}")
    odd = np.float32([[1.0, np.nan, 2.0, 0.5], [0.0, -np.inf, 3.0, 1.0],
                      [-np.inf] * 4, [np.inf, 0.0, 1.0, 2.0]])
    got = model.softmax_dim(torch.from_numpy(odd).to(dev), 1).cpu().numpy()
    want = oracle.softmax_dim(odd, 1)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    close(got[fin], want[fin], "nan / inf rows")
    with pytest.raises(Exception):
        model.softmax_dim(torch.zeros((2, 0), device=dev), 1)


@pytest.mark.gpu
@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (2, 2, 2), (1, 128, 37), (33, 47, 129),
                                   (64, 128, 2304), (5, 0, 3)])
def test_gpu_matmul_transpose_mul_scalar_bit_exact(torch_dev, m, k, n):
    """matmul in the naive loop's serial order, transpose and mul_scalar give
    the oracle's bits (crates/ndarray-backend/src/lib.rs:208-219, :270-281,
    :747-756)."""
    torch, dev = torch_dev
    rng = np.random.default_rng(m * 1000 + k * 10 + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    ta, tb = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    y = model.matmul(ta, tb).cpu().numpy()
    assert np.array_equal(y.view(np.uint32), oracle.matmul(a, b).view(np.uint32))
    if k:
        assert np.array_equal(model.transpose(ta).cpu().numpy(), a.T)
        assert np.array_equal(model.mul_scalar(ta, -0.0883883).cpu().numpy(),
                              oracle.mul_scalar(a, -0.0883883))


@pytest.mark.gpu
def test_gpu_per_head_recipe_on_device_ops_matches_paged_decode(torch_dev):
    """The reference's per-head recipe (tape_transformer.rs:87-139: q K^T,
    * scale, softmax, @ V) composed from the device ops equals the oracle's
    paged decode attention over the same K / V within 1e-4 / 1e-3."""
    torch, dev = torch_dev
    rng = np.random.default_rng(11)
    hq, hkv, d, bs = 8, 2, 64, 16
    ctx = np.array([1, 37, 300], np.int32)
    need = (ctx + bs - 1) // bs
    nb = int(need.sum())
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.full((len(ctx), int(need.max())), -1, np.int32)
    o = 0
    for i, c in enumerate(need):
        tables[i, :c] = perm[o:o + c]
        o += c
    kp = rng.standard_normal((nb, hkv, bs, d)).astype(np.float32)
    vp = rng.standard_normal((nb, hkv, bs, d)).astype(np.float32)
    q = rng.standard_normal((len(ctx), hq, d)).astype(np.float32)
    scale = 1 / math.sqrt(d)
    want = oracle.decode_attention(q, kp, vp, tables, ctx, scale)
    for b, L in enumerate(ctx):
        rows = tables[b, np.arange(L) // bs], np.arange(L) % bs
        for h in range(hq):
            g = h // (hq // hkv)
            k = np.ascontiguousarray(kp[rows[0], g, rows[1]])  # [L, D]
            v = np.ascontiguousarray(vp[rows[0], g, rows[1]])
            tq = torch.from_numpy(q[b, h][None]).to(dev)
            s = model.matmul(tq, model.transpose(torch.from_numpy(k).to(dev)))
            p = model.softmax_dim(model.mul_scalar(s, scale), 1)
            out = model.matmul(p, torch.from_numpy(v).to(dev)).cpu().numpy()[0]
            diff = np.abs(out - want[b, h])
            assert ((diff <= 1e-4) | (diff <= 1e-3 * np.abs(want[b, h]))).all(), (b, h)


@pytest.mark.gpu
def test_gpu_decoder_pool_size_does_not_change_tokens(dev):
    """The same weights in decoders of max_seq 1024 and 128 (64 and 8 KV
    blocks per layer, other attention grids): tokens equal the CPU
    decoder's in both, logits within 1e-4 / 1e-3 of it and of each other."""
    from tests.gpu_util import say
    say("decoder: max_seq 1024 and 128")
    params = model.init_params(model.config(), seed=5, std=0.02)
    prompt = np.random.default_rng(6).integers(0, 1000, 20).astype(np.int32)
    want, wlg = oracle.decoder_generate(oracle.decoder_config(), params, prompt, 40, logits=True)
    outs = []
    for max_seq in (1024, 128):
        dec = model.Decoder(model.config(max_seq=max_seq), params)
        toks, lg = dec.generate(prompt, 40, logits=True)
        assert toks.tolist() == want.tolist(), max_seq
        np.testing.assert_allclose(lg, wlg, atol=1e-4, rtol=1e-3)
        outs.append(lg)
    np.testing.assert_allclose(outs[0], outs[1], atol=1e-4, rtol=1e-3)


@pytest.mark.gpu
def test_gpu_decoder_config0_tokens_equal_oracle(dev):
    """weights N(0, 0.02) from seed 0, prompt of 32 ids from seed
    0, 64 greedy tokens through paged KV (16-token blocks): token-identical
    to the CPU oracle; logits within the fp32 attention tolerance."""
    from tests.gpu_util import say
    say("decoder configs[0] end to end")
    cfg = model.config()
    params = model.init_params(cfg, seed=0, std=0.02)
    prompt = np.random.default_rng(0).integers(0, 1000, 32).astype(np.int32)
    dec = model.Decoder(cfg, params)
    toks, lg = dec.generate(prompt, 64, logits=True)
    want, wlg = oracle.decoder_generate(oracle.decoder_config(), params, prompt, 64, logits=True)
    srt = np.sort(wlg, axis=1)
    margin = float((srt[:, -1] - srt[:, -2]).min())
    say(f"min top-1/top-2 logit margin {margin:.3e}, max |dlogit| {np.abs(lg - wlg).max():.2e}")
    assert toks.tolist() == want.tolist()
    np.testing.assert_allclose(lg, wlg, atol=1e-4, rtol=1e-3)
    # a second call reuses the pools (blocks come back in a different order)
    # and replays the captured launch sequence
    toks2 = dec.generate(prompt, 64)
    assert toks2.tolist() == want.tolist()
    # replays with other data of the same shape, a new shape (a new capture),
    # and the first shape again: every call equals the CPU decoder's
    rng = np.random.default_rng(1)
    for n_prompt, n_new in ((32, 64), (32, 64), (5, 20), (32, 64)):
        p2 = rng.integers(0, 1000, n_prompt).astype(np.int32)
        got = dec.generate(p2, n_new)
        ref = oracle.decoder_generate(oracle.decoder_config(), params, p2, n_new)
        assert got.tolist() == ref.tolist(), (n_prompt, n_new)


def test_config0_token_fixture_is_the_oracles():
    """tests/golden/config0_tokens.txt (read by the Rust crate's test) holds
    the oracle decoder's configs[0] tokens."""
    import os
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import make_config0_tokens as mk
    prompt, want = mk.tokens()
    rows = {}
    for line in open(os.path.join(os.path.dirname(__file__), "golden", "config0_tokens.txt")):
        if not line.startswith("#"):
            key, *vals = line.split()
            rows[key] = [int(v) for v in vals]
    assert rows["prompt"] == prompt.tolist() and rows["tokens"] == want.tolist()
