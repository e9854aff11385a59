"""Writes tests/golden/decode_small.npz: seeded inputs for paged decode
attention plus expected outputs computed in float64 by numpy (gather +
einsum + softmax), a formulation independent of the oracle's loops.

Run from the repo root: python tests/golden/make_golden.py
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    rng = np.random.default_rng(20261201)
    B, hq, hkv, d, bs, nb = 3, 4, 2, 32, 16, 12
    ctx = np.array([1, 17, 40], np.int32)
    k = rng.standard_normal((nb, hkv, bs, d)).astype(np.float32)
    v = rng.standard_normal((nb, hkv, bs, d)).astype(np.float32)
    q = rng.standard_normal((B, hq, d)).astype(np.float32)
    tables = np.full((B, 3), -1, np.int32)
    perm = rng.permutation(nb).astype(np.int32)
    tables[0, :1] = perm[0:1]
    tables[1, :2] = perm[1:3]
    tables[2, :3] = perm[3:6]
    scale = np.float32(1.0 / np.sqrt(d))
    out = np.zeros((B, hq, d))
    g = hq // hkv
    for b in range(B):
        L = int(ctx[b])
        pos = np.arange(L)
        blk = tables[b, pos // bs]
        K = k[blk, :, pos % bs, :].astype(np.float64)
        V = v[blk, :, pos % bs, :].astype(np.float64)
        for h in range(hq):
            s = K[:, h // g, :] @ q[b, h].astype(np.float64) * float(scale)
            p = np.exp(s - s.max())
            out[b, h] = (p / p.sum()) @ V[:, h // g, :]
    np.savez(os.path.join(HERE, "decode_small.npz"), q=q, k_pool=k, v_pool=v, tables=tables,
             ctx_lens=ctx, scale=scale, expected=out)


if __name__ == "__main__":
    main()
