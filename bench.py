"""Paged-KV decode attention benchmark on one MI355X.

Workload (the configuration the metric is quoted
on): Llama-3-8B attention shape, batch 64, 32 query heads, 8 KV heads
(GQA 4:1), head_dim 128, block size 16, bf16 KV pools with fp32
accumulation, context lengths U[512, 4096] (seed 2), random block tables,
q/K/V ~ N(0, 1), scale 1/sqrt(128).

One step = one decode token for the batch through the attention of a
32-layer stack: 32 calls of rkv_decode_attention, each on its own layer's
KV pool (32 x ~604 MB, far beyond the 256 MB Infinity Cache, so every call
streams from HBM).  GEMMs of the model are not part of this path.

Prints one JSON line.  value = algorithmic bytes / time over the whole step
(both split-K passes and launch gaps); roofline.achieved = algorithmic
bytes / the partition kernel's own average duration, from HIP events
recorded on the launch stream around every launch in the timed region.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
B, HQ, HKV, D, BS = 64, 32, 8, 128, 16
CTX_LO, CTX_HI, SEED = 512, 4096, 2


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--layers", type=int, default=32)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-threads", type=int, default=0, help="0: min(nproc, 16)")
    p.add_argument("--copy-only", action="store_true",
                   help="only run the 1 GiB device copy (calibrates rocprof FETCH/WRITE_SIZE)")
    return p.parse_args()


def build_workload(torch, dev, n_layers):
    import numpy as np
    rng = np.random.default_rng(SEED)
    ctx = rng.integers(CTX_LO, CTX_HI + 1, size=B).astype(np.int32)
    need = (ctx.astype(np.int64) + BS - 1) // BS
    nb = int(need.sum())
    mbs = CTX_HI // BS
    g = torch.Generator(device=dev).manual_seed(SEED)
    layers = []
    for _ in range(n_layers):
        k = torch.randn((nb, HKV, BS, D), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((nb, HKV, BS, D), generator=g, device=dev).to(torch.bfloat16)
        q = torch.randn((B, HQ, D), generator=g, device=dev)
        perm = torch.randperm(nb, generator=g, device=dev).to(torch.int32)
        tables = torch.full((B, mbs), -1, dtype=torch.int32, device=dev)
        o = 0
        for b in range(B):
            n = int(need[b])
            tables[b, :n] = perm[o:o + n]
            o += n
        layers.append((q, k, v, tables))
    ctx_d = torch.from_numpy(ctx).to(dev)
    return layers, ctx, ctx_d, nb, mbs


def algorithmic_bytes(ctx):
    n = len(ctx)
    kv_bytes = sum(int(L) * HKV * D * 2 * 2 for L in ctx)           # K and V, bf16
    qo = n * HQ * D * 4 * 2                                          # q read + out write
    tables = sum((int(L) + BS - 1) // BS for L in ctx) * 4 + n * 4   # block ids + ctx lens
    return kv_bytes + qo + tables


def copy_bandwidth(torch, dev, nbytes=2 << 30, reps=10):
    """Device-to-device copy GB/s (read + write) as the achievable HBM rate."""
    a = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=dev).normal_()
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    return 2 * nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9


def cpu_baseline(torch, layers, ctx, threads):
    """The C oracle (a restatement of the reference's CPU semantics) on a
    bounded sample: layer 0 of the workload, all 64 sequences, timed with
    `threads` POSIX threads, plus one single-thread pass over 4 sequences."""
    import numpy as np
    import oracle
    q, k, v, tables = layers[0]
    qh = q.cpu().numpy()
    kh = k.cpu().view(torch.int16).numpy().view(np.uint16)
    vh = v.cpu().view(torch.int16).numpy().view(np.uint16)
    th = tables.cpu().numpy()
    scale = 1.0 / math.sqrt(D)
    oracle.decode_attention(qh[:1], kh, vh, th[:1], ctx[:1], scale)  # load + warm
    reps, t_mt = 0, 0.0
    while reps < 3 and t_mt < 10.0:
        t0 = time.perf_counter()
        oracle.decode_attention(qh, kh, vh, th, ctx, scale, n_threads=threads)
        t_mt += time.perf_counter() - t0
        reps += 1
    t0 = time.perf_counter()
    oracle.decode_attention(qh[:4], kh, vh, th[:4], ctx[:4], scale)
    t_st = time.perf_counter() - t0
    mt_gbps = algorithmic_bytes(ctx) * reps / t_mt / 1e9
    st_gbps = algorithmic_bytes(ctx[:4]) / t_st / 1e9
    return {
        "value": round(mt_gbps, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": (f"oracle/rkv_oracle.c decode attention, layer 0 of the workload (64 seqs, "
                   f"bf16 pool), {reps} call(s) on {threads} threads in {t_mt:.2f} s; "
                   f"single thread on 4 seqs: {st_gbps:.3f} GB/s"),
        "single_thread_GBps": round(st_gbps, 4),
        "tokens_per_s_32_layers": round(B * reps / (t_mt * 32), 3),
    }


def traffic_from_profiles():
    p = os.path.join(ROOT, "profiles", "decode_config2_traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f)
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the path would shard by sequence or KV head, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import torch
    from rustral_amd import kv

    dev = torch.device("cuda:0")
    if args.copy_only:
        gbps = copy_bandwidth(torch, dev, nbytes=1 << 30, reps=5)
        print(json.dumps({"copy_bytes": 1 << 30, "reps": 6, "copy_GBps": round(gbps, 1)}))
        return
    layers, ctx, ctx_d, nb, mbs = build_workload(torch, dev, args.layers)
    n_layers = len(layers)
    max_ctx = mbs * BS
    ws = torch.empty(kv.workspace_bytes(B, HQ, D, max_ctx), dtype=torch.uint8, device=dev)
    outs = [torch.empty((B, HQ, D), device=dev) for _ in range(n_layers)]
    scale = 1.0 / math.sqrt(D)

    def call(i, passes):
        q, k, v, t = layers[i]
        kv.decode_attention(q, k, v, t, ctx_d, scale, max_context=max_ctx, out=outs[i],
                            workspace=ws, passes=passes)

    for _ in range(args.warmup):
        for i in range(n_layers):
            call(i, "both")
    torch.cuda.synchronize()

    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    marks = [[(ev(), ev(), ev()) for _ in range(n_layers)] for _ in range(args.steps)]
    start, stop = ev(), ev()
    torch.cuda.synchronize()
    start.record()
    for s in range(args.steps):
        for i in range(n_layers):
            a, m, e = marks[s][i]
            a.record()
            call(i, "partitions")
            m.record()
            call(i, "merge")
            e.record()
    stop.record()
    torch.cuda.synchronize()

    total_ms = start.elapsed_time(stop)
    ms_step = total_ms / args.steps
    part_ms = [a.elapsed_time(m) for row in marks for (a, m, e) in row]
    merge_ms = [m.elapsed_time(e) for row in marks for (a, m, e) in row]
    avg_part_us = 1e3 * sum(part_ms) / len(part_ms)
    avg_merge_us = 1e3 * sum(merge_ms) / len(merge_ms)
    bytes_call = algorithmic_bytes(ctx)
    call_us = 1e3 * ms_step / n_layers
    value = bytes_call / (call_us * 1e-6) / 1e9
    achieved = bytes_call / (avg_part_us * 1e-6) / 1e9
    tokens_per_s = B / (ms_step * 1e-3) * (n_layers / 32)

    traffic = traffic_from_profiles()
    copy_gbps = copy_bandwidth(torch, dev)
    cpu = None
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or min(os.cpu_count() or 1, 16)
        cpu = cpu_baseline(torch, layers, ctx, threads)

    line = {
        "metric": "paged-KV decode attention GB/s (% of HBM peak); decode tokens/s at batch 64",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,1) q/K/V, seeded contexts U[512,4096], random block tables",
        "config": {"workload": "configs[2] paged decode attention, Llama-3-8B layer shape",
                   "batch": B, "num_q_heads": HQ, "num_kv_heads": HKV, "head_dim": D,
                   "block_size": BS, "kv_dtype": "bf16", "accumulate": "fp32",
                   "context": [CTX_LO, CTX_HI], "mean_context": float(ctx.mean()),
                   "layers_per_step": n_layers, "step": "one decode token: 32 attention calls"},
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBPS, 2),
        "decode_tokens_per_s_b64": round(tokens_per_s, 1),
        "us_per_call": round(call_us, 2),
        "partition_kernel_us": round(avg_part_us, 2),
        "merge_kernel_us": round(avg_merge_us, 2),
        "algorithmic_bytes_per_call": bytes_call,
        "measured_copy_GBps": round(copy_gbps, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "kernel": "decode_stream_kernel<bf16, D=128, G=4> (one wave per 256-token partition)",
                     "traffic": traffic},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
