"""Paged-KV decode attention benchmark on one MI355X.

Workload (benchmark configs[2], the configuration the metric is quoted
on): Llama-3-8B attention shape, batch 64, 32 query heads, 8 KV heads
(GQA 4:1), head_dim 128, block size 16, bf16 KV pools with fp32
accumulation, context lengths U[512, 4096] (seed 2), random block tables,
q/K/V ~ N(0, 1), scale 1/sqrt(128).

One step = one decode token for the batch through the attention of a
32-layer stack: 32 calls of rkv_decode_attention, each on its own layer's
KV pool (32 x ~604 MB, far beyond the 256 MB Infinity Cache, so every call
streams from HBM).  GEMMs of the model are not part of this path.

Prints one JSON line.  value = algorithmic bytes / time over the whole step
(both split-K passes and the gaps between launches), the 32 calls of a step
captured once in a HIP graph and replayed K times, as a serving loop replays
its step; roofline.achieved = algorithmic bytes / the partition kernel's own
average duration, from HIP events recorded on the launch stream around every
launch of a second, eagerly launched timed region of K steps.

Other workloads (--workload config0|config1|config3|config4|prefill) print
their own line.
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
    p.add_argument("--workload", default="config2",
                   choices=["config0", "config1", "config2", "config3", "config4", "prefill",
                            "decode_q", "device_step", "ceilings", "store_variants",
                            "patterns_1byte"],
                   help="config2 (default): the headline decode line; the others print "
                        "their own line (benchmark configs[0], [1], [3], [4])")
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


def read_bandwidth(torch, dev, nbytes=2 << 30, reps=10):
    """Flat nontemporal read GB/s of rustral_amd/ceiling's stream kernel: the
    achievable rate for a read-only kernel such as the decode (None if that
    measurement library is not built)."""
    try:
        from rustral_amd import ceiling as C
        C.lib()
    except (ImportError, OSError):
        return None
    a = torch.full((nbytes // 4,), 1, dtype=torch.int32, device=dev)
    sink = torch.zeros(16, dtype=torch.int32, device=dev)
    C.read(torch, a, sink)
    ms = _timed(torch, lambda: C.read(torch, a, sink), reps)
    del a
    return nbytes / (ms * 1e-3) / 1e9


def cpu_baseline(torch, layers, ctx, threads):
    """The C oracle (a restatement of the reference's CPU semantics) on a
    bounded sample: layer 0 of the workload, all 64 sequences, timed with
    `threads` POSIX threads, repeated for about 10 s, plus one single-thread
    pass over 4 sequences."""
    import numpy as np
    import oracle
    q, k, v, tables = layers[0]
    qh = q.cpu().numpy()
    kh = k.cpu().view(torch.int16).numpy().view(np.uint16)
    vh = v.cpu().view(torch.int16).numpy().view(np.uint16)
    th = tables.cpu().numpy()
    scale = 1.0 / math.sqrt(D)
    oracle.decode_attention(qh[:1], kh, vh, th[:1], ctx[:1], scale)  # load + warm
    reps, t_mt, calls = 0, 0.0, []
    while t_mt < 10.0 and reps < 500:  # about 10 s of CPU work
        t0 = time.perf_counter()
        oracle.decode_attention(qh, kh, vh, th, ctx, scale, n_threads=threads)
        calls.append(time.perf_counter() - t0)
        t_mt += calls[-1]
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
        "call_ms_stats": stats([1e3 * t for t in calls]),
    }


def stats(samples):
    """mean / p50 / std / CI95 of per-step times (ms), in the spirit of the
    reference bench's schema-v2 statistics (crates/bench/src/lib.rs:236-310):
    CI95 = mean +- 1.96 std / sqrt(n)."""
    import numpy as np
    a = np.asarray(samples, np.float64)
    n = len(a)
    sd = float(a.std(ddof=1)) if n > 1 else 0.0
    h = 1.96 * sd / math.sqrt(n) if n > 1 else 0.0
    return {"n": n, "mean": round(float(a.mean()), 5), "p50": round(float(np.median(a)), 5),
            "std": round(sd, 5), "min": round(float(a.min()), 5), "max": round(float(a.max()), 5),
            "ci95": [round(float(a.mean()) - h, 5), round(float(a.mean()) + h, 5)]}


def machine(torch):
    """Where the numbers were taken: GPU, HIP / torch versions, host CPU."""
    cpu_model = None
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    cpu_model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    props = torch.cuda.get_device_properties(0)
    return {"gpu": torch.cuda.get_device_name(0), "gcn_arch": getattr(props, "gcnArchName", None),
            "compute_units": props.multi_processor_count,
            "gpu_memory_GiB": round(props.total_memory / 2**30, 1),
            "hip": torch.version.hip, "torch": torch.__version__, "cpu_model": cpu_model,
            "host_nproc": os.cpu_count(), "host_cpus_usable": affinity,
            "timestamp_utc": time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime())}


def traffic_from_profiles():
    """HBM bytes per launch of the partition kernel from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs (scaled by a 1 GiB copy)."""
    p = os.path.join(ROOT, "profiles", "decode_config2_traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    return None


# ---- the other benchmark configs (one JSON line each; not the headline) -----------

def _timed(torch, fn, reps, settle_s=0.05):
    """Average ms of fn() over reps calls, HIP events on the current stream,
    after untimed rounds of reps calls for at least settle_s seconds (the
    clock takes ~15 ms of sustained load to settle)."""
    t0 = time.perf_counter()
    while True:
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= settle_s:
            break
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def _line(metric, value, unit, ms, args, dtype, config, **extra):
    d = {"metric": metric, "value": round(value, 2), "unit": unit, "n_gpus": 1,
         "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
         "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
         "data": "synthetic", "config": config}
    d["pct_hbm_peak"] = round(100 * value / HBM_PEAK_GBPS, 2) if unit == "GB/s" else None
    d.update(extra)
    return d


def run_config0(torch, dev, args):
    """the 2-layer decoder (d 128, 4 heads of 32, MLP 512, vocab
    1000, fp32) with weights N(0, 0.02) from seed 0, a 32-id prompt (seed 0)
    and 64 greedy tokens through the paged fp32 KV cache, batch 1.  One step =
    one generated token (the prompt is fed one token per step as well, so a
    generation is 95 decoder steps).  The cpu_baseline leg runs the C oracle's
    decoder on the same weights and prompt; its tokens must equal the GPU's."""
    import numpy as np
    from rustral_amd import model
    cfg = model.config()
    params = model.init_params(cfg, seed=0, std=0.02)
    prompt = np.random.default_rng(0).integers(0, 1000, 32).astype(np.int32)
    n_new = 64
    dec = model.Decoder(cfg, params)
    for _ in range(max(args.warmup, 1)):
        toks = dec.generate(prompt, n_new)
    reps = max(args.steps // 4, 3)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        toks = dec.generate(prompt, n_new)       # synchronizes at its end
    dt = (time.perf_counter() - t0) / reps
    gpu_tps = n_new / dt
    cpu = None
    if not args.no_cpu_baseline:
        import oracle
        ocfg = oracle.decoder_config()
        t0 = time.perf_counter()
        want = oracle.decoder_generate(ocfg, params, prompt, n_new)
        cdt = time.perf_counter() - t0
        cpu = {"value": round(n_new / cdt, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"oracle/rkv_oracle.c decoder, the same 32-id prompt + {n_new} greedy "
                         f"tokens, one thread, {cdt:.3f} s",
               "tokens_equal_gpu": bool(np.array_equal(want, toks))}
    steps = len(prompt) + n_new - 1
    # the serving engine on the same model: the prompt in one prefill step,
    # then decode steps; one request alone, then 64 requests at max batch 16
    def serve(n_req, max_batch):
        rng = np.random.default_rng(10)
        prompts = [rng.integers(0, 1000, 32).astype(np.int32) for _ in range(n_req)]
        best = None
        for _ in range(2):
            eng = model.Engine(cfg, params, num_blocks=n_req * 6 + 8, max_batch_size=max_batch)
            ids = [eng.submit(p_, n_new) for p_ in prompts]
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            n_steps = eng.run()
            dt_ = time.perf_counter() - t0
            ntok = sum(len(eng.generated(i)) for i in ids)
            del eng
            if best is None or dt_ < best[0]:
                best = (dt_, ntok, n_steps)
        return {"requests": n_req, "max_batch": max_batch, "steps": best[2],
                "tokens": best[1], "seconds": round(best[0], 4),
                "tokens_per_s": round(best[1] / best[0], 1)}
    engine = {"batch1": serve(1, 1), "batch16_64_requests": serve(64, 16)}
    return _line("configs[0] greedy decode tokens/s, batch 1 (GPU tokens checked against the CPU decoder)",
                 gpu_tps, "tokens/s", 1e3 * dt / steps, args, "fp32",
                 {"workload": "configs[0] tiny decoder, 2 layers, d_model 128, 4 heads x 32, "
                              "d_ff 512, vocab 1000, paged fp32 KV (16-token blocks)",
                  "prompt": int(len(prompt)), "generated": n_new, "batch": 1},
                 ms_per_generation=round(1e3 * dt, 3), decoder_steps=steps,
                 us_per_decoder_step=round(1e6 * dt / steps, 2), serving_engine=engine,
                 cpu_baseline=cpu)


def run_config1(torch, dev, args):
    """32 layers, Hkv 8, D 128, BS 16; 64 sequences each appending
    one token per step into a 65,536-block pool (random tables), gather of
    contexts U[512, 4096].  bf16: 32 distinct layer pools (128 GiB);
    fp32: 16 layer pools (128 GiB; 32 would not fit next to the rest)."""
    import numpy as np
    from rustral_amd import kv
    rng = np.random.default_rng(1)
    nb, hkv, bs, d, B = 65536, HKV, BS, D, 64
    ctx = rng.integers(512, 4096 + 1, size=B).astype(np.int32)
    need = (ctx + bs - 1) // bs
    mbs = 4096 // bs + 1
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.full((B, mbs), -1, np.int32)
    o = 0
    for b in range(B):
        n = int(need[b]) + 2                       # room for 16+ appended tokens
        tables[b, :n] = perm[o:o + n]
        o += n
    res = {}
    for dtype, n_layers in (("bf16", 32), ("f32", 16)):
        tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
        s_pool = 2 if dtype == "bf16" else 4
        kp = torch.empty((n_layers, nb, hkv, bs, d), dtype=tdt, device=dev)
        vp = torch.empty_like(kp)
        g = torch.Generator(device=dev).manual_seed(1)
        # N_SRC distinct per-step sources (512 MiB for bf16, beyond the 256 MB
        # Infinity Cache), so a step's fp32 K/V rows come from HBM
        n_src = 32
        kns = torch.randn((n_src, n_layers, B, hkv, d), generator=g, device=dev)
        vns = torch.randn((n_src, n_layers, B, hkv, d), generator=g, device=dev)
        kn, vn = kns[0], vns[0]
        steps = max(args.steps, 4)
        slot_sets = []
        for s in range(16):                       # token L + s of every sequence, cycled
            p = ctx + s
            slot_sets.append(torch.from_numpy(
                tables[np.arange(B), p // bs].astype(np.int64) * bs + p % bs).to(dev))
        it = iter(range(10 ** 9))
        def app():
            i = next(it)
            kv.append(kp, vp, kns[i % n_src], vns[i % n_src], slot_sets[i % len(slot_sets)])
        for _ in range(args.warmup):
            app()
        ms_app = _timed(torch, app, steps)
        app_bytes = n_layers * B * hkv * d * 2 * (4 + s_pool) + B * 8
        # n_src per-step launches (sources rotating, slots cycling) captured
        # once in a HIP graph and replayed, as a serving loop captures its
        # step (no host launch cost)
        def steps_of_graph():
            for j in range(n_src):
                kv.append(kp, vp, kns[j], vns[j], slot_sets[j % len(slot_sets)])
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            steps_of_graph()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            steps_of_graph()
        graph.replay()
        ms_graph = _timed(torch, graph.replay, max(steps // 4, 3)) / n_src
        del graph
        # bulk: the 16 steps' tokens (1024 per layer) in one launch, as a
        # prefill or a batch of queued steps would append them
        knb = torch.randn((n_layers, 16 * B, hkv, d), generator=g, device=dev)
        vnb = torch.randn_like(knb)
        bulk_slots = torch.cat(slot_sets)
        def bulk():
            kv.append(kp, vp, knb, vnb, bulk_slots)
        bulk()
        ms_bulk = _timed(torch, bulk, steps)
        bulk_bytes = n_layers * 16 * B * hkv * d * 2 * (4 + s_pool) + 16 * B * 8
        del knb, vnb
        gt, gc = torch.from_numpy(tables).to(dev), torch.from_numpy(ctx).to(dev)
        offs = torch.from_numpy(np.concatenate([[0], np.cumsum(ctx.astype(np.int64) * hkv * d)[:-1]])).to(dev)
        total = int(ctx.astype(np.int64).sum()) * hkv * d
        outs = {}
        for odt, name in ((tdt, "same"), (torch.float32, "f32")):
            if name == "f32" and dtype == "f32":
                continue
            ko = torch.empty(total, dtype=odt, device=dev)
            vo = torch.empty_like(ko)
            li = iter(range(10 ** 9))
            def gat():
                l = next(li) % n_layers
                kv.gather(kp[l], vp[l], gt, gc, out_offsets=offs, out_total=total, k_out=ko, v_out=vo)
            gat()
            ms_g = _timed(torch, gat, n_layers)
            s_out = 2 if odt == torch.bfloat16 else 4
            g_bytes = int(ctx.astype(np.int64).sum()) * hkv * d * 2 * (s_pool + s_out) + int(need.sum()) * 4
            outs[name] = {"us_per_call": round(1e3 * ms_g, 2), "GBps": round(g_bytes / (ms_g * 1e-3) / 1e9, 1),
                          "bytes_per_call": g_bytes}
        res[dtype] = {"layers": n_layers, "append": {
            "us_per_step": round(1e3 * ms_app, 2), "bytes_per_step": app_bytes,
            "GBps": round(app_bytes / (ms_app * 1e-3) / 1e9, 1)},
            "append_graph": {"us_per_step": round(1e3 * ms_graph, 2), "bytes_per_step": app_bytes,
                             "GBps": round(app_bytes / (ms_graph * 1e-3) / 1e9, 1)},
            "append_bulk_16_steps": {"us_per_launch": round(1e3 * ms_bulk, 2),
                                     "bytes_per_launch": bulk_bytes,
                                     "GBps": round(bulk_bytes / (ms_bulk * 1e-3) / 1e9, 1)},
            "gather_packed": outs}
        del kp, vp, kn, vn, kns, vns
        torch.cuda.empty_cache()
    a = res["bf16"]["append_graph"]
    gb = res["bf16"]["gather_packed"]["same"]
    return _line("KV append GB/s per step (64 tokens x 32 layers, one launch per step; 32 steps "
                 "with distinct sources replayed from a HIP graph), bf16 pool", a["GBps"],
                 "GB/s", a["us_per_step"] / 1e3, args, "bf16",
                 {"workload": "configs[1] KV append + gather microbench", "num_kv_heads": hkv,
                  "head_dim": d, "block_size": bs, "pool_blocks": nb, "sequences": B,
                  "context": [512, 4096]},
                 gather_GBps_bf16=gb["GBps"],
                 append_eager_GBps_bf16=res["bf16"]["append"]["GBps"],
                 append_bulk_GBps_bf16=res["bf16"]["append_bulk_16_steps"]["GBps"], results=res)


def _decode_layers(torch, dev, B, lo, hi, seed, n_layers):
    import numpy as np
    rng = np.random.default_rng(seed)
    ctx = rng.integers(lo, hi + 1, size=B).astype(np.int32)
    need = (ctx.astype(np.int64) + BS - 1) // BS
    nb = int(need.sum())
    mbs = (hi + BS - 1) // BS
    g = torch.Generator(device=dev).manual_seed(seed)
    layers = []
    for _ in range(n_layers):
        k = torch.randn((nb, HKV, BS, D), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((nb, HKV, BS, D), generator=g, device=dev).to(torch.bfloat16)
        q = torch.randn((B, HQ, D), generator=g, device=dev)
        perm = torch.randperm(nb, generator=g, device=dev).to(torch.int32).cpu().numpy()
        tab = np.full((B, mbs), -1, np.int32)
        o = 0
        for b in range(B):
            tab[b, :need[b]] = perm[o:o + need[b]]
            o += int(need[b])
        layers.append((q, k, v, torch.from_numpy(tab).to(dev)))
    return layers, ctx, torch.from_numpy(ctx).to(dev), mbs * BS


def run_config3(torch, dev, args):
    """B 8, Hq 32, Hkv 8, D 128, bf16, contexts U[16384, 65536],
    permuted blocks; two-pass split-K.  8 layer pools (10.7 GB) rotate so no
    call re-reads the previous one's bytes from the 256 MB Infinity Cache."""
    from rustral_amd import kv
    n_layers = 8
    layers, ctx, ctx_d, max_ctx = _decode_layers(torch, dev, 8, 16384, 65536, 3, n_layers)
    ws = torch.empty(kv.workspace_bytes(8, HQ, D, max_ctx), dtype=torch.uint8, device=dev)
    out = torch.empty((8, HQ, D), device=dev)
    scale = 1.0 / math.sqrt(D)
    it = iter(range(10 ** 9))
    def call():
        q, k, v, t = layers[next(it) % n_layers]
        kv.decode_attention(q, k, v, t, ctx_d, scale, max_context=max_ctx, out=out, workspace=ws)
    for _ in range(max(args.warmup, 1) * n_layers):
        call()
    reps = max(args.steps, 4) * n_layers
    ms = _timed(torch, call, reps)
    nbytes = algorithmic_bytes(ctx)
    gbps = nbytes / (ms * 1e-3) / 1e9
    return _line("long-context split-K paged decode GB/s (% of HBM peak)", gbps, "GB/s", ms, args,
                 "bf16", {"workload": "configs[3] long-context split-K decode", "batch": 8,
                          "num_q_heads": HQ, "num_kv_heads": HKV, "head_dim": D, "block_size": BS,
                          "context": [16384, 65536], "mean_context": float(ctx.mean())},
                 us_per_call=round(1e3 * ms, 2), algorithmic_bytes_per_call=nbytes,
                 calls_timed=reps)


def prefill_bytes_flops(n_new, ctx, hq=HQ, hkv=HKV, d=D, s_kv=2):
    """Algorithmic bytes and flops of one causal prefill call.  Bytes: q read
    and out written (fp32), each sequence's K and V read once per KV head
    (positions 0 .. ctx-1), block ids, q_start and ctx_lens.  Flops: 2 * D per
    (query, key) pair for QK^T and again for PV, over the causal pairs."""
    nbytes = flops = 0
    for n, L in zip(n_new, ctx):
        n, L = int(n), int(L)
        nbytes += n * hq * d * 4 * 2 + L * hkv * d * 2 * s_kv + ((L + BS - 1) // BS) * 4 + 8
        pairs = sum(L - n + i + 1 for i in range(n))
        flops += pairs * hq * d * 4
    return nbytes, flops


def run_prefill(torch, dev, args):
    """Causal prefill over the paged pool at configs[4]'s admission shape: 25
    sequences x 128 new prompt tokens (ctx == 128), Hq 32, Hkv 8, D 128, bf16
    pool, 32 layers (distinct q and pools per layer), one call per layer.  A
    second figure: a chunked prefill of 512 new tokens after 3584 cached ones
    for 8 sequences (the compute-heavy end).  us_per_call times the layers'
    calls back to back (events around each burst of 32, as a forward pass
    keeps the GPU busy); us_per_call_events_each times each call between
    events of its own (the GPU idles between calls)."""
    import numpy as np
    from rustral_amd import kv
    g = torch.Generator(device=dev).manual_seed(7)

    def layers_for(n_new, ctx, n_layers):
        need = [(int(L) + BS - 1) // BS for L in ctx]
        nb = int(sum(need))
        qs = torch.from_numpy(np.concatenate([[0], np.cumsum(n_new)]).astype(np.int32)).to(dev)
        cl = torch.from_numpy(np.asarray(ctx, np.int32)).to(dev)
        out = []
        for _ in range(n_layers):
            k = torch.randn((nb, HKV, BS, D), generator=g, device=dev).to(torch.bfloat16)
            v = torch.randn((nb, HKV, BS, D), generator=g, device=dev).to(torch.bfloat16)
            q = torch.randn((int(sum(n_new)), HQ, D), generator=g, device=dev)
            perm = torch.randperm(nb, generator=g, device=dev).to(torch.int32).cpu().numpy()
            t = np.full((len(ctx), max(need)), -1, np.int32)
            o = 0
            for b, n in enumerate(need):
                t[b, :n] = perm[o:o + n]
                o += n
            out.append((q, k, v, torch.from_numpy(t).to(dev), torch.empty_like(q)))
        return out, qs, cl

    def measure(n_new, ctx, n_layers, reps_per_layer):
        layers, qs, cl = layers_for(n_new, ctx, n_layers)
        mq = int(max(n_new))
        it = iter(range(10 ** 9))
        def call():
            q, k, v, t, o = layers[next(it) % n_layers]
            kv.prefill_attention(q, k, v, t, qs, cl, 1.0 / math.sqrt(D), max_q_len=mq, out=o)
        # untimed passes over the layers for at least 50 ms: the clock
        # takes ~15 ms of this load to settle (admissions: 27-33 us per call
        # over the first ~15 bursts of 32, 26.0 after)
        t_warm = time.perf_counter()
        while True:
            for _ in range(n_layers):
                call()
            torch.cuda.synchronize()
            if time.perf_counter() - t_warm > 0.05:
                break
        # the layers' calls back to back, events around each burst (the GPU
        # stays busy, as in a forward pass), then with events around each call
        bursts = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(reps_per_layer)]
        torch.cuda.synchronize()
        for a, e in bursts:
            a.record()
            for _ in range(n_layers):
                call()
            e.record()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(n_layers * reps_per_layer)]
        torch.cuda.synchronize()
        for a, e in ev:
            a.record()
            call()
            e.record()
        torch.cuda.synchronize()
        us_burst = 1e3 * sum(a.elapsed_time(e) for a, e in bursts) / (len(bursts) * n_layers)
        us_each = 1e3 * sum(a.elapsed_time(e) for a, e in ev) / len(ev)
        del layers
        torch.cuda.empty_cache()
        return us_burst, us_each

    n_adm = np.full(25, 128, np.int32)
    us_adm, us_adm_each = measure(n_adm, n_adm, 32, max(args.steps // 4, 3))
    b_adm, f_adm = prefill_bytes_flops(n_adm, n_adm)
    n_chk = np.full(8, 512, np.int32)
    c_chk = np.full(8, 4096, np.int32)
    us_chk, us_chk_each = measure(n_chk, c_chk, 8, max(args.steps // 4, 3))
    b_chk, f_chk = prefill_bytes_flops(n_chk, c_chk)
    gbps = b_adm / (us_adm * 1e-6) / 1e9
    return _line("causal prefill over paged KV GB/s (configs[4] admissions: 25 x 128 tokens)", gbps,
                 "GB/s", us_adm / 1e3, args, "bf16",
                 {"workload": "paged causal prefill, configs[4] admission shape", "sequences": 25,
                  "new_tokens": 128, "context": 128, "num_q_heads": HQ, "num_kv_heads": HKV,
                  "head_dim": D, "block_size": BS, "layers": 32},
                 us_per_call=round(us_adm, 2), us_per_call_events_each=round(us_adm_each, 2),
                 algorithmic_bytes_per_call=b_adm,
                 flops_per_call=f_adm, tflops=round(f_adm / (us_adm * 1e-6) / 1e12, 2),
                 chunked_512_after_3584={"sequences": 8, "us_per_call": round(us_chk, 2),
                                         "us_per_call_events_each": round(us_chk_each, 2),
                                         "bytes": b_chk, "flops": f_chk,
                                         "GBps": round(b_chk / (us_chk * 1e-6) / 1e9, 1),
                                         "tflops": round(f_chk / (us_chk * 1e-6) / 1e12, 2)})


def run_decode_q(torch, dev, args):
    """configs[2]'s decode (B64, Hq32, Hkv8, D128, contexts U[512, 4096], seed
    2, 32 layer pools) over 1-byte pools: int8 and OCP fp8 e4m3 with one fp32
    scale per (token, KV head) row, filled by the quantizing append from
    N(0, 1) rows.  A step (32 calls) is replayed from a HIP graph as in the
    headline line.  Bytes per call: the bytes and scales of K and V once, q
    in, out, block ids, lengths.  Beside it, per format: the dequantizing
    gather of a layer into the packed fp32 KVCache layout (bytes and scales
    read, fp32 written) and the quantizing append of 1,024 tokens into 32
    layers in one launch (fp32 rows read, bytes and scales written)."""
    import numpy as np
    from rustral_amd import kv
    rng = np.random.default_rng(SEED)
    ctx = rng.integers(CTX_LO, CTX_HI + 1, size=B).astype(np.int32)
    need = (ctx.astype(np.int64) + BS - 1) // BS
    nb = int(need.sum())
    mbs = CTX_HI // BS
    g = torch.Generator(device=dev).manual_seed(SEED)
    ctx_d = torch.from_numpy(ctx).to(dev)
    slots = torch.arange(nb * BS, dtype=torch.int64, device=dev)
    scale = 1.0 / math.sqrt(D)
    res = {}
    for fmt in ("int8", "fp8"):
        layers = []
        for _ in range(32):
            kp = torch.empty((nb, HKV, BS, D), dtype=torch.uint8, device=dev)
            vp = torch.empty_like(kp)
            ks = torch.empty((nb, HKV, BS), dtype=torch.float32, device=dev)
            vs = torch.empty_like(ks)
            kn = torch.randn((nb * BS, HKV, D), generator=g, device=dev)
            vn = torch.randn((nb * BS, HKV, D), generator=g, device=dev)
            kv.append_q(kp, vp, ks, vs, kn, vn, slots, fmt)
            del kn, vn
            q = torch.randn((B, HQ, D), generator=g, device=dev)
            perm = torch.randperm(nb, generator=g, device=dev).to(torch.int32)
            t = torch.full((B, mbs), -1, dtype=torch.int32, device=dev)
            o = 0
            for b in range(B):
                t[b, :int(need[b])] = perm[o:o + int(need[b])]
                o += int(need[b])
            layers.append((q, kp, vp, ks, vs, t, torch.empty_like(q)))
        ws = torch.empty(kv.workspace_bytes(B, HQ, D, CTX_HI), dtype=torch.uint8, device=dev)

        def step():
            for (q, kp, vp, ks, vs, t, o) in layers:
                kv.decode_attention_q(q, kp, vp, ks, vs, t, ctx_d, scale, fmt,
                                      max_context=CTX_HI, out=o, workspace=ws)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(max(args.warmup, 1)):
                step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        graph.replay()
        ms = _timed(torch, graph.replay, args.steps)
        del graph
        nbytes = (int(ctx.astype(np.int64).sum()) * HKV * (D + 4) * 2 + B * HQ * D * 4 * 2
                  + int(need.sum()) * 4 + B * 4)
        us = 1e3 * ms / 32
        res[fmt] = {"us_per_call": round(us, 2), "bytes_per_call": nbytes,
                    "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                    "decode_tokens_per_s_b64": round(B / (ms * 1e-3), 1)}
        # a model's per-layer order: the new token's quantizing append, then
        # the attention, per layer -- as two launches, and fused (the new
        # row rewrites position ctx - 1 of every sequence on each replay)
        last = torch.from_numpy((ctx.astype(np.int64) - 1)).to(dev)
        kn1 = torch.randn((B, HKV, D), generator=g, device=dev)
        vn1 = torch.randn((B, HKV, D), generator=g, device=dev)
        slot_l = [(t[torch.arange(B, device=dev), last // BS].to(torch.int64) * BS + last % BS)
                  for (_, _, _, _, _, t, _) in layers]

        def step_pl():
            for (q, kp, vp, ks, vs, t, o), sl in zip(layers, slot_l):
                kv.append_q(kp, vp, ks, vs, kn1, vn1, sl, fmt)
                kv.decode_attention_q(q, kp, vp, ks, vs, t, ctx_d, scale, fmt,
                                      max_context=CTX_HI, out=o, workspace=ws)

        def step_fu():
            for (q, kp, vp, ks, vs, t, o) in layers:
                kv.decode_attention_append_q(q, kp, vp, ks, vs, kn1, vn1, t, ctx_d, scale, fmt,
                                             max_context=CTX_HI, out=o, workspace=ws)
        app1 = B * HKV * D * (4 + 1) * 2 + B * HKV * 4 * 2
        for name, fn in (("per_layer_append_q_then_decode_q", step_pl),
                         ("per_layer_fused_append_decode_q", step_fu)):
            fn()
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                fn()
            gr.replay()
            m2 = _timed(torch, gr.replay, args.steps)
            del gr
            res[fmt][name] = {"ms_per_step": round(m2, 4),
                              "GBps": round(32 * (nbytes + app1) / (m2 * 1e-3) / 1e9, 1)}
        # dequantizing gather into the packed KVCache layout, one layer per
        # call, rotating over the 32 layer pools
        n_tok = int(ctx.astype(np.int64).sum())
        offs = torch.from_numpy(np.concatenate(
            [[0], np.cumsum(ctx.astype(np.int64) * HKV * D)[:-1]])).to(dev)
        total = n_tok * HKV * D
        ko = torch.empty(total, dtype=torch.float32, device=dev)
        vo = torch.empty_like(ko)
        li = iter(range(10 ** 9))

        def gat():
            _, kp, vp, ks, vs, t, _ = layers[next(li) % len(layers)]
            kv.gather_q(kp, vp, ks, vs, t, ctx_d, fmt, out_offsets=offs, out_total=total,
                        k_out=ko, v_out=vo)
        gat()
        ms_g = _timed(torch, gat, len(layers))
        g_bytes = n_tok * HKV * 2 * ((D + 4) + 4 * D) + int(need.sum()) * 4 + B * 4
        res[fmt]["gather_packed"] = {"us_per_call": round(1e3 * ms_g, 2), "bytes_per_call": g_bytes,
                                     "GBps": round(g_bytes / (ms_g * 1e-3) / 1e9, 1)}
        del layers, ws, ko, vo
        torch.cuda.empty_cache()
        # quantizing append: 16 decode steps' tokens (1,024) into all 32
        # layers of a 4,096-block pool set in one launch, distinct random slots
        nl, nba, n_app = 32, 4096, 16 * B
        akp = torch.empty((nl, nba, HKV, BS, D), dtype=torch.uint8, device=dev)
        avp = torch.empty_like(akp)
        aks = torch.empty((nl, nba, HKV, BS), dtype=torch.float32, device=dev)
        avs = torch.empty_like(aks)
        akn = torch.randn((nl, n_app, HKV, D), generator=g, device=dev)
        avn = torch.randn_like(akn)
        aslots = torch.randperm(nba * BS, generator=g, device=dev)[:n_app].contiguous()

        def app():
            kv.append_q(akp, avp, aks, avs, akn, avn, aslots, fmt)
        app()
        ms_a = _timed(torch, app, max(args.steps, 5))
        a_bytes = nl * n_app * HKV * 2 * (4 * D + D + 4) + n_app * 8
        res[fmt]["append_bulk_16_steps"] = {"us_per_launch": round(1e3 * ms_a, 2),
                                            "bytes_per_launch": a_bytes,
                                            "GBps": round(a_bytes / (ms_a * 1e-3) / 1e9, 1)}
        del akp, avp, aks, avs, akn, avn
        torch.cuda.empty_cache()
    r = res["int8"]
    return _line("paged-KV decode over int8 pools GB/s (configs[2] shape); tokens/s at batch 64",
                 r["GBps"], "GB/s", 32 * r["us_per_call"] / 1e3, args, "int8",
                 {"workload": "configs[2] decode shape over 1-byte KV pools (int8, fp8 e4m3) "
                              "with per-row fp32 scales", "batch": B, "num_q_heads": HQ,
                  "num_kv_heads": HKV, "head_dim": D, "block_size": BS,
                  "context": [CTX_LO, CTX_HI], "layers_per_step": 32},
                 results=res)


def run_config4(torch, dev, args):
    """continuous-batching step mix.  256 running sequences with
    contexts U[1, 8192] (seed 4) in 32 layer pools of 84,000 blocks (bf16,
    176 GB), blocks handed out one at a time round-robin by the host block
    manager (so finished sequences leave holes).  One step: 10% of the
    sequences finish (blocks freed), the block manager plans the relocation of
    25% of the live blocks (rkv_bm_plan_relocation: highest ids first into the
    longest runs of free ids, both sides ascending) and copy_blocks moves them
    (all layers, K and V, one launch), 10% new sequences are admitted with 128-token prefills
    appended in bulk (one launch for all layers) and run through causal
    prefill attention (one call per layer), then one decode token for every
    running sequence: append (one launch) + 32 decode-attention calls.
    Hq = 32 (GQA 4:1) is assumed; the benchmark configuration does not state it.  One untimed
    and four timed steps: every step replaces 10% of the sequences by
    128-token ones, so a longer run drifts away from the configuration's
    context distribution U[1, 8192]."""
    import numpy as np
    from rustral_amd import kv
    from rustral_amd.serving import PagedCache
    rng = np.random.default_rng(4)
    n_layers, nblk, B, pre = 32, 84000, 256, 128
    n_turn = B // 10                                 # finish / admit per step
    blk_bytes = HKV * BS * D * 2
    kp = torch.empty((n_layers, nblk, HKV, BS, D), dtype=torch.bfloat16, device=dev)
    vp = torch.empty_like(kp)
    kp.fill_(0.01), vp.fill_(-0.01)
    cache = PagedCache(BS, nblk)
    ctx = {i: int(c) for i, c in enumerate(rng.integers(1, 8192 + 1, size=B))}
    next_id = B
    pending = {i: -(-c // BS) for i, c in ctx.items()}
    while pending:                                   # round-robin, one block at a time
        for i in list(pending):
            assert cache.allocate(i, BS) is not None
            pending[i] -= 1
            if pending[i] == 0:
                del pending[i]
    g = torch.Generator(device=dev).manual_seed(4)
    kn_pre = torch.randn((n_layers, n_turn * pre, HKV, D), generator=g, device=dev)
    vn_pre = torch.randn_like(kn_pre)
    kn_dec = torch.randn((n_layers, B, HKV, D), generator=g, device=dev)
    vn_dec = torch.randn_like(kn_dec)
    q = torch.randn((B, HQ, D), generator=g, device=dev)
    out = torch.empty_like(q)
    q_pre = torch.randn((n_turn * pre, HQ, D), generator=g, device=dev)
    out_pre = torch.empty_like(q_pre)
    d_qs = torch.arange(0, (n_turn + 1) * pre, pre, dtype=torch.int32, device=dev)
    d_cpre = torch.full((n_turn,), pre, dtype=torch.int32, device=dev)
    ws = torch.empty(kv.workspace_bytes(B, HQ, D, 8192 + 64 * BS), dtype=torch.uint8, device=dev)
    scale = 1.0 / math.sqrt(D)
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    steps = []
    warmup, timed = 1, 4
    for step in range(warmup + timed):
        t_host = time.perf_counter()
        ids = sorted(ctx)
        n_fin = n_turn
        for i in rng.choice(ids, size=n_fin, replace=False).tolist():
            cache.free(i)
            del ctx[i]
        live = sum(len(cache.table(i)) for i in ctx)
        pairs = cache.plan_relocation(live // 4)
        assert len(pairs) == live // 4, "the pool is too small to relocate 25% of the live blocks"
        admitted = []
        for _ in range(n_fin):
            cache.allocate(next_id, pre)
            ctx[next_id] = pre
            admitted.append(next_id)
            next_id += 1
        slots_pre = np.concatenate([np.asarray(cache.table(i), np.int64)[np.arange(pre) // BS] * BS
                                    + np.arange(pre) % BS for i in admitted])
        tab_pre = cache.fill_tables(admitted, pre // BS)
        ids = sorted(ctx)
        for i in ids:                                  # room for the decode token
            cache.reserve(i, ctx[i] + 1)
        mb = max(len(cache.table(i)) for i in ids)
        tables = cache.fill_tables(ids, mb)
        cl = np.array([ctx[i] for i in ids], np.int32)
        pos = cl.astype(np.int64)
        slots_dec = tables[np.arange(len(ids)), pos // BS].astype(np.int64) * BS + pos % BS
        for i in ids:
            ctx[i] += 1
        cl_after = cl + 1
        d_pairs = torch.from_numpy(pairs.astype(np.int32)).to(dev)
        d_spre = torch.from_numpy(slots_pre).to(dev)
        d_tpre = torch.from_numpy(tab_pre).to(dev)
        d_sdec = torch.from_numpy(slots_dec).to(dev)
        d_tab = torch.from_numpy(tables).to(dev)
        d_ctx = torch.from_numpy(cl_after).to(dev)
        n_pre = len(slots_pre)
        torch.cuda.synchronize()
        t_host = time.perf_counter() - t_host
        e = [ev() for _ in range(6)]
        e[0].record()
        if len(pairs):
            kv.copy_blocks(kp, vp, d_pairs)
        e[1].record()
        kv.append(kp, vp, kn_pre, vn_pre, d_spre)
        e[2].record()
        for l in range(n_layers):
            kv.prefill_attention(q_pre, kp[l], vp[l], d_tpre, d_qs, d_cpre, scale, max_q_len=pre,
                                 out=out_pre)
        e[5].record()
        nb_ = len(ids)
        assert nb_ == B and n_pre == n_turn * pre
        kv.append(kp, vp, kn_dec, vn_dec, d_sdec)
        e[3].record()
        for l in range(n_layers):
            kv.decode_attention(q, kp[l], vp[l], d_tab, d_ctx, scale,
                                max_context=mb * BS, out=out, workspace=ws)
        e[4].record()
        torch.cuda.synchronize()
        if step < warmup:
            continue
        ms = [e[0].elapsed_time(e[1]), e[1].elapsed_time(e[2]), e[2].elapsed_time(e[5]),
              e[5].elapsed_time(e[3]), e[3].elapsed_time(e[4])]
        copy_b = len(pairs) * n_layers * 2 * blk_bytes * 2
        pre_b = n_pre * n_layers * HKV * D * 2 * (4 + 2) + n_pre * 8
        dec_app_b = nb_ * n_layers * HKV * D * 2 * (4 + 2) + nb_ * 8
        attn_b = n_layers * (int(cl_after.astype(np.int64).sum()) * HKV * D * 2 * 2
                             + nb_ * HQ * D * 8 + int(sum(-(-c // BS) for c in cl_after)) * 4)
        pa_b, pa_f = prefill_bytes_flops(np.full(n_turn, pre), np.full(n_turn, pre))
        steps.append(dict(pairs=len(pairs), live_blocks=live, prefill_tokens=n_pre,
                          running=nb_, ms=ms, host_ms=1e3 * t_host,
                          bytes=[copy_b, pre_b, n_layers * pa_b, dec_app_b, attn_b]))
    n = len(steps)
    ms = np.array([s["ms"] for s in steps]).mean(0)
    by = np.array([s["bytes"] for s in steps], np.float64).mean(0)
    gbps = by / (ms * 1e-3) / 1e9
    total_ms = float(ms.sum())
    total_gbps = float(by.sum() / (total_ms * 1e-3) / 1e9)
    comps = ["copy_blocks", "prefill_append", "prefill_attention_32_layers", "decode_append",
             "decode_attention_32_layers"]
    import types
    return _line("continuous-batching step GB/s (copy + prefill append/attention + decode "
                 "append/attention)", total_gbps,
                 "GB/s", total_ms, types.SimpleNamespace(steps=timed, warmup=warmup), "bf16",
                 {"workload": "configs[4] continuous-batching step mix", "running": B,
                  "layers": n_layers, "num_q_heads": HQ, "num_kv_heads": HKV, "head_dim": D,
                  "block_size": BS, "pool_blocks_per_layer": nblk, "prefill": pre,
                  "relocated_share_of_live_blocks": round(float(np.mean(
                      [s["pairs"] / s["live_blocks"] for s in steps])), 4)},
                 components={c: {"ms": round(float(m), 3), "GBps": round(float(gb), 1),
                                 "bytes": int(b)} for c, m, gb, b in zip(comps, ms, gbps, by)},
                 decode_tokens_per_s=round(float(np.mean([s["running"] for s in steps]))
                                           / (total_ms * 1e-3), 1),
                 steps_detail=[{k: v for k, v in s.items() if k != "bytes"} for s in steps[:n]])


def run_device_step(torch, dev, args):
    """configs[2]'s batch (64 sequences, contexts U[512,4096]) stepping one
    decode token at a time through a 32-layer attention stack with the cache
    managed on the device: per step rkv_dbm_reserve (tables grow at block
    boundaries), rkv_dbm_slot_mapping, one multi-layer rkv_append of the new
    token's K/V, rkv_dbm_batch_tables and 32 rkv_decode_attention calls, the
    context lengths advanced in place -- captured once in a HIP graph and
    replayed, no host work per step.  Blocks were handed out by growing all
    sequences one block at a time (interleaved, as a running batch grows),
    so each sequence's blocks are spread through the pool."""
    import numpy as np
    from rustral_amd import kv
    n_layers = args.layers
    steps, warm = args.steps, args.warmup
    rng = np.random.default_rng(SEED)
    ctx = rng.integers(CTX_LO, CTX_HI + 1, size=B).astype(np.int32)
    grow = 3 * (warm + steps + 1)          # three step variants run one after the other
    mbs = (CTX_HI + grow + BS - 1) // BS
    nb = int(((ctx + grow + BS - 1) // BS).sum()) + 64
    g = torch.Generator(device=dev).manual_seed(SEED)
    kpool = torch.empty((n_layers, nb, HKV, BS, D), dtype=torch.bfloat16, device=dev)
    vpool = torch.empty_like(kpool)
    for l in range(n_layers):  # N(0, 1) values, one layer at a time (bf16)
        kpool[l].copy_(torch.randn((nb, HKV, BS, D), generator=g, device=dev))
        vpool[l].copy_(torch.randn((nb, HKV, BS, D), generator=g, device=dev))
    dbm = kv.DeviceBlockManager(nb, BS, B, mbs, device=dev)
    slots = torch.arange(B, dtype=torch.int32, device=dev)
    # interleaved growth: round r gives every sequence with more than r
    # blocks its block r
    for r in range(int(((ctx + BS - 1) // BS).max())):
        dbm.reserve(slots, torch.as_tensor(np.minimum(ctx, (r + 1) * BS), dtype=torch.int32))
    nf, err = dbm.status()
    assert err == 0
    q = [torch.randn((B, HQ, D), generator=g, device=dev) for _ in range(n_layers)]
    k_new = torch.randn((n_layers, B, HKV, D), generator=g, device=dev)
    v_new = torch.randn((n_layers, B, HKV, D), generator=g, device=dev)
    lens = torch.as_tensor(ctx, dtype=torch.int32, device=dev)   # tokens cached before the step
    nlen = torch.empty_like(lens)
    max_ctx = mbs * BS
    ws = torch.empty(kv.workspace_bytes(B, HQ, D, max_ctx), dtype=torch.uint8, device=dev)
    outs = [torch.empty((B, HQ, D), device=dev) for _ in range(n_layers)]
    scale = 1.0 / math.sqrt(D)

    def step():
        torch.add(lens, 1, out=nlen)
        dbm.reserve(slots, nlen)
        sm = dbm.slot_mapping(slots, lens)      # the new token's position = old length
        kv.append(kpool, vpool, k_new, v_new, sm)
        tab = dbm.batch_tables(slots, mbs)
        for l in range(n_layers):
            kv.decode_attention(q[l], kpool[l], vpool[l], tab, nlen, scale, max_context=max_ctx,
                                out=outs[l], workspace=ws)
        lens.copy_(nlen)

    def step_per_layer():
        # a model's order: layer l's K/V exist only after layer l's
        # projections, so each layer appends its own row, then attends
        torch.add(lens, 1, out=nlen)
        dbm.reserve(slots, nlen)
        sm = dbm.slot_mapping(slots, lens)
        tab = dbm.batch_tables(slots, mbs)
        for l in range(n_layers):
            kv.append(kpool[l], vpool[l], k_new[l], v_new[l], sm)
            kv.decode_attention(q[l], kpool[l], vpool[l], tab, nlen, scale, max_context=max_ctx,
                                out=outs[l], workspace=ws)
        lens.copy_(nlen)

    def step_fused():
        # the same order with the append fused into each layer's decode
        torch.add(lens, 1, out=nlen)
        dbm.reserve(slots, nlen)
        tab = dbm.batch_tables(slots, mbs)
        for l in range(n_layers):
            kv.decode_attention_append(q[l], kpool[l], vpool[l], k_new[l], v_new[l], tab, nlen,
                                       scale, max_context=max_ctx, out=outs[l], workspace=ws)
        lens.copy_(nlen)

    stream = torch.cuda.Stream(device=dev)
    base = 0

    def run_graph(fn):
        nonlocal base
        stream.wait_stream(torch.cuda.current_stream(dev))
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                fn()
        torch.cuda.synchronize(dev)
        lens.copy_(torch.as_tensor(ctx + base, dtype=torch.int32))  # the capture runs nothing
        torch.cuda.synchronize(dev)
        for _ in range(warm):
            graph.replay()
        mid = ctx + base + warm + 1 + steps // 2   # mean context over the timed steps
        t = _timed(torch, graph.replay, steps)
        base += warm + steps
        del graph
        return t, mid

    ms, ctx_mid = run_graph(step)
    ms_pl, ctx_pl = run_graph(step_per_layer)
    ms_fu, ctx_fu = run_graph(step_fused)
    nf_end, err = dbm.status()
    assert err == 0, "device block manager reported an error during the bench"
    attn_bytes = algorithmic_bytes(ctx_mid) * n_layers
    app_bytes = n_layers * B * HKV * D * 2 * (4 + 2) + B * 8
    tok_s = B / (ms / 1e3)
    variants = {
        "per_layer_append_then_decode": {
            "ms_per_step": round(ms_pl, 4), "tokens_per_s": round(B / (ms_pl / 1e3), 1),
            "step_GBps": round((algorithmic_bytes(ctx_pl) * n_layers + app_bytes)
                               / (ms_pl / 1e3) / 1e9, 1)},
        "per_layer_fused_append_decode": {
            "ms_per_step": round(ms_fu, 4), "tokens_per_s": round(B / (ms_fu / 1e3), 1),
            "step_GBps": round((algorithmic_bytes(ctx_fu) * n_layers + app_bytes)
                               / (ms_fu / 1e3) / 1e9, 1)}}
    dbm.close()
    return _line("decode step tokens/s at batch 64 with the KV cache managed on the device "
                 "(configs[2] shape, 32 layers)", tok_s, "tokens/s", ms, args, "bf16",
                 {"workload": "configs[2] decode steps, device-resident block tables",
                  "batch": B, "num_q_heads": HQ, "num_kv_heads": HKV, "head_dim": D,
                  "block_size": BS, "layers": n_layers, "context": [CTX_LO, CTX_HI],
                  "step": "reserve + slot mapping + append (all layers) + batch tables + "
                          "32 decode calls, one HIP graph replay"},
                 step_GBps=round((attn_bytes + app_bytes) / (ms / 1e3) / 1e9, 1),
                 attention_bytes_per_step=attn_bytes, append_bytes_per_step=app_bytes,
                 free_blocks_after=nf_end, step_variants=variants)


def run_ceilings(torch, dev, args):
    """What HBM streams at on this part for the access patterns of the
    paged-KV kernels (rustral_amd/ceiling: kernels that move bytes and do
    nothing else): flat nontemporal read, flat write and flat copy of 4 GiB;
    32 KiB block copies inside a 4 GiB pool (a quarter of its blocks: random
    pairs, sorted by destination, sequential runs); and the decode kernel's
    own loads at configs[2] (its grid, block tables and ring of tiles over
    the bench's 32 layer pools) timed beside the decode partition kernel on
    the same pools."""
    import numpy as np
    from rustral_amd import ceiling as C
    from rustral_amd import kv
    reps = max(args.steps // 4, 5)
    res = {}

    def rate(fn, moved):
        fn()
        ms = _timed(torch, fn, reps)
        return {"GBps": round(moved / (ms * 1e-3) / 1e9, 1), "us": round(1e3 * ms, 2),
                "bytes": int(moved)}

    sink = torch.zeros(16, dtype=torch.int32, device=dev)
    nbytes = 4 << 30
    a = torch.full((nbytes // 4,), 1, dtype=torch.int32, device=dev)
    b = torch.empty_like(a)
    res["read_flat"] = rate(lambda: C.read(torch, a, sink), nbytes)
    res["write_flat"] = rate(lambda: C.write(torch, b), nbytes)
    res["copy_flat"] = rate(lambda: C.copy(torch, a, b), 2 * nbytes)
    blk = 32768                                   # a bf16 block, Hkv 8, D 128
    nblk = nbytes // blk
    npairs = nblk // 4
    rng = np.random.default_rng(3)
    perm = rng.permutation(nblk).astype(np.int32)
    pairs = {"random": np.stack([perm[:npairs], perm[npairs:2 * npairs]], 1)}
    pairs["sorted_dst"] = pairs["random"][np.argsort(pairs["random"][:, 1], kind="stable")]
    pairs["sequential"] = np.stack([np.arange(nblk - 1, nblk - 1 - npairs, -1),
                                    np.arange(npairs)], 1).astype(np.int32)
    for name, pr in pairs.items():
        pd = torch.from_numpy(np.ascontiguousarray(pr, dtype=np.int32)).to(dev)
        res[f"block_copy_{name}"] = rate(lambda: C.block_copy(torch, a, pd, blk), 2 * npairs * blk)
    del a, b
    torch.cuda.empty_cache()
    layers, ctx, ctx_d, nb, mbs = build_workload(torch, dev, args.layers)
    n_layers, max_ctx = len(layers), mbs * BS
    parts = (max_ctx + 639) // 640
    kv_bytes = sum(int(L) * HKV * D * 2 * 2 for L in ctx)

    def stream_all():
        for q, k, v, t in layers:
            C.tile_stream(torch, k, v, t, ctx_d, sink, parts)
    st = rate(stream_all, kv_bytes * n_layers)
    res["decode_tile_stream"] = {"GBps": st["GBps"], "us_per_layer": round(st["us"] / n_layers, 2),
                                 "kv_bytes_per_layer": kv_bytes}
    # the same pattern at the partition shape the decode call picks for this
    # workload (768 tokens: 8 waves of 6 tiles), which the decode kernel below
    # runs
    pick = kv.partition_size_for(B, HQ, HKV, D, kv._lib.RKV_BF16, max_ctx)
    shape = {640: (10, 4), 768: (6, 8), 1280: (10, 8)}.get(pick)
    if shape:
        parts_p = (max_ctx + pick - 1) // pick

        def stream_pick():
            for q, k, v, t in layers:
                C.tile_stream_shape(torch, k, v, t, ctx_d, sink, parts_p, *shape)
        sp = rate(stream_pick, kv_bytes * n_layers)
        res["decode_tile_stream_picked_shape"] = {
            "partition_tokens": pick, "tiles_per_wave": shape[0], "waves": shape[1],
            "GBps": sp["GBps"], "us_per_layer": round(sp["us"] / n_layers, 2)}
    ws = torch.empty(kv.workspace_bytes(B, HQ, D, max_ctx), dtype=torch.uint8, device=dev)
    out = torch.empty((B, HQ, D), device=dev)
    scale = 1.0 / math.sqrt(D)

    def decode_all():
        for q, k, v, t in layers:
            kv.decode_attention(q, k, v, t, ctx_d, scale, max_context=max_ctx, out=out,
                                workspace=ws, passes="partitions")
    dp = rate(decode_all, kv_bytes * n_layers)
    res["decode_partition_kernel"] = {"GBps_kv": dp["GBps"],
                                      "us_per_layer": round(dp["us"] / n_layers, 2)}
    ratio = round(dp["GBps"] / st["GBps"], 4)
    ratio_pick = (round(dp["GBps"] / res["decode_tile_stream_picked_shape"]["GBps"], 4)
                  if "decode_tile_stream_picked_shape" in res else None)
    # the same shape, tables and q over 1-byte pools (int8 bytes, fp32 row scales)
    g8 = torch.Generator(device=dev).manual_seed(SEED + 1)
    layers8 = []
    for i in range(n_layers):
        q, k, v, t = layers[i]
        shp = tuple(k.shape)
        layers[i] = None                          # the bf16 pools are not needed any more
        kp = torch.randint(0, 256, shp, generator=g8, dtype=torch.uint8, device=dev)
        vp = torch.randint(0, 256, shp, generator=g8, dtype=torch.uint8, device=dev)
        ks = torch.rand(shp[:3], generator=g8, device=dev) * 0.02
        vs = torch.rand(shp[:3], generator=g8, device=dev) * 0.02
        layers8.append((q, kp, vp, ks, vs, t))
    del layers
    torch.cuda.empty_cache()
    kv8_bytes = sum(int(L) * HKV * (D + 4) * 2 for L in ctx)

    def stream8_all():
        for q, kp, vp, ks, vs, t in layers8:
            C.tile_stream(torch, kp, vp, t, ctx_d, sink, parts, k_scale=ks, v_scale=vs)
    st8 = rate(stream8_all, kv8_bytes * n_layers)
    res["decode_tile_stream_1byte"] = {"GBps": st8["GBps"],
                                       "us_per_layer": round(st8["us"] / n_layers, 2),
                                       "kv_bytes_per_layer": kv8_bytes}

    def decode8_all():
        for q, kp, vp, ks, vs, t in layers8:
            kv.decode_attention_q(q, kp, vp, ks, vs, t, ctx_d, scale, "int8",
                                  max_context=max_ctx, out=out, workspace=ws)
    d8 = rate(decode8_all, kv8_bytes * n_layers)
    res["decode_int8_both_passes"] = {"GBps_kv": d8["GBps"],
                                      "us_per_layer": round(d8["us"] / n_layers, 2)}
    return _line("HBM ceilings of the paged-KV access patterns: the decode kernel's loads "
                 "streamed with no arithmetic (configs[2])", st["GBps"], "GB/s",
                 st["us"] / n_layers / 1e3, args, "bf16",
                 {"workload": "stream kernels of rustral_amd/ceiling; configs[2] pools for the "
                              "decode pattern", "flat_bytes": nbytes, "block_bytes": blk,
                  "block_pairs": npairs, "layers": n_layers},
                 decode_partition_over_stream=ratio,
                 decode_partition_over_stream_same_shape=ratio_pick,
                 decode_int8_over_stream_1byte=round(d8["GBps"] / st8["GBps"], 4), results=res)


def run_patterns_1byte(torch, dev, args):
    """The int8 decode's load pattern and variants of it, loads only
    (rustral_amd/ceiling `tile_stream_1b`), timed beside the int8 decode call
    (partition kernel and merge) on configs[2]'s shape over 32 layers of
    1-byte pools: the pattern as the decode kernel reads it (2 KiB (block,
    head) tiles plus the fp32 row scales), without the scales, two or four KV
    heads per wave, a partition-major grid, and the K and V row scales in a
    128-byte line after each K tile."""
    import numpy as np
    from rustral_amd import ceiling as C
    from rustral_amd import kv
    reps = max(args.steps // 4, 5)
    rng = np.random.default_rng(SEED)
    ctx = rng.integers(CTX_LO, CTX_HI + 1, size=B).astype(np.int32)
    need = (ctx.astype(np.int64) + BS - 1) // BS
    nb = int(need.sum())
    mbs = CTX_HI // BS
    ctx_d = torch.from_numpy(ctx).to(dev)
    g = torch.Generator(device=dev).manual_seed(SEED + 2)
    layers = []
    for _ in range(args.layers):
        kp = torch.randint(0, 256, (nb, HKV, BS, D), generator=g, dtype=torch.uint8, device=dev)
        vp = torch.randint(0, 256, (nb, HKV, BS, D), generator=g, dtype=torch.uint8, device=dev)
        kc = torch.randint(0, 256, (nb, HKV, BS * D + 128), generator=g, dtype=torch.uint8,
                           device=dev)
        ks = torch.rand((nb, HKV, BS), generator=g, device=dev) * 0.02
        vs = torch.rand((nb, HKV, BS), generator=g, device=dev) * 0.02
        q = torch.randn((B, HQ, D), generator=g, device=dev)
        perm = torch.randperm(nb, generator=g, device=dev).to(torch.int32)
        t = torch.full((B, mbs), -1, dtype=torch.int32, device=dev)
        o = 0
        for b in range(B):
            t[b, :int(need[b])] = perm[o:o + int(need[b])]
            o += int(need[b])
        layers.append((q, kp, vp, kc, ks, vs, t))
    n_layers = len(layers)
    parts = (CTX_HI + 639) // 640
    tokens = int(ctx.astype(np.int64).sum())
    with_scales = tokens * HKV * (D + 4) * 2
    sink = torch.zeros(16, dtype=torch.int32, device=dev)

    def rate(fn, moved):
        fn()
        ms = _timed(torch, fn, reps)
        return {"GBps": round(moved * n_layers / (ms * 1e-3) / 1e9, 1),
                "us_per_layer": round(1e3 * ms / n_layers, 2), "bytes_per_layer": int(moved)}

    res = {}
    for name in C.TILE_STREAM_1B:
        moved = tokens * HKV * D * 2 if name == "no_scales" else with_scales

        def fn(name=name):
            for q, kp, vp, kc, ks, vs, t in layers:
                C.tile_stream_1b(torch, kc if name == "scales_after_k_tile" else kp, vp, t, ctx_d,
                                 sink, parts, name, nb, HKV, k_scale=ks, v_scale=vs)
        res[name] = rate(fn, moved)
    out = torch.empty((B, HQ, D), device=dev)
    ws = torch.empty(kv.workspace_bytes(B, HQ, D, CTX_HI), dtype=torch.uint8, device=dev)
    scale = 1.0 / math.sqrt(D)

    def decode_all():
        for q, kp, vp, kc, ks, vs, t in layers:
            kv.decode_attention_q(q, kp, vp, ks, vs, t, ctx_d, scale, "int8",
                                  max_context=CTX_HI, out=out, workspace=ws)
    res["decode_int8_call"] = rate(decode_all, with_scales)
    base = res["row_scales"]
    return _line("int8 decode load pattern and variants, loads only (configs[2] shape)",
                 base["GBps"], "GB/s", base["us_per_layer"] / 1e3, args, "u8",
                 {"workload": "tile_stream_1b of rustral_amd/ceiling over 32 layers of 1-byte "
                              "pools, configs[2] contexts", "layers": n_layers,
                  "partitions": parts, "tokens": tokens},
                 decode_call_over_pattern=round(res["decode_int8_call"]["GBps"] / base["GBps"], 4),
                 results=res)


def run_store_variants(torch, dev, args):
    """Write and copy ceilings from writers other than the library's own
    stream kernels: hipMemsetD32Async (eager), torch's fill_ and zero_,
    hipMemcpyAsync device to device, and the store variants of
    rustral_amd/ceiling (default or nontemporal store policy, one or two
    16-byte vectors per lane, grid-stride interleave or one contiguous chunk
    per workgroup, grids from one workgroup per CU to one-shot) over 4 GiB
    buffers.  Rates count the bytes moved (a copy: read + written)."""
    import ctypes
    from rustral_amd import ceiling as C
    reps = max(args.steps // 4, 5)
    nbytes = 4 << 30
    a = torch.full((nbytes // 4,), 1, dtype=torch.int32, device=dev)
    b = torch.empty_like(a)
    hip = ctypes.CDLL("libamdhip64.so.7")           # torch's runtime, already loaded
    hip.hipMemsetD32Async.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t,
                                      ctypes.c_void_p]
    hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                   ctypes.c_void_p]
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def rate(fn, moved):
        fn()
        ms = _timed(torch, fn, reps)
        return round(moved / (ms * 1e-3) / 1e9, 1)

    def memset():
        assert hip.hipMemsetD32Async(b.data_ptr(), 0x3F800000, nbytes // 4, stream) == 0

    def memcpy():
        assert hip.hipMemcpyAsync(b.data_ptr(), a.data_ptr(), nbytes, 3, stream) == 0  # D2D
    res = {"independent": {
        "hipMemsetD32Async": rate(memset, nbytes),
        "torch_fill_": rate(lambda: b.fill_(7), nbytes),
        "torch_zero_": rate(lambda: b.zero_(), nbytes),
        "hipMemcpyAsync_d2d": rate(memcpy, 2 * nbytes),
        "torch_copy_": rate(lambda: b.copy_(a), 2 * nbytes),
    }}
    grids = [256, 512, 1024, 2048, 8192, 65536, 131072]   # the last two: one round per
                                                           # workgroup for 2 / 1 vectors a lane
    names = {0: "default", 1: "nt", 2: "x2", 3: "nt_x2", 4: "chunk", 5: "nt_chunk",
             6: "x2_chunk", 7: "nt_x2_chunk"}
    res["write"] = {f"{names[v]}@{g}": rate(lambda: C.write_var(torch, b, g, v), nbytes)
                    for v in range(8) for g in grids}
    # work per workgroup: unr x 4 KiB, one round each (2 GiB launches as
    # torch's fill makes them, and 4 GiB), or grid-stride over 1-8 per CU
    half = b[: b.numel() // 2]
    sink = torch.zeros(16, dtype=torch.int32, device=dev)
    res["read"] = {}
    for unr in (1, 2, 4, 8, 16):
        res["read"][f"unr{unr}_oneshot"] = rate(lambda: C.read_unr(torch, a, sink, unr), nbytes)
        for g in (1024, 4096):
            res["read"][f"unr{unr}@{g}"] = rate(lambda: C.read_unr(torch, a, sink, unr, g), nbytes)
    for unr in (1, 2, 4, 8):
        res["write"][f"unr{unr}_oneshot"] = rate(lambda: C.write_unr(torch, b, unr), nbytes)
        res["write"][f"unr{unr}_oneshot_2GiB"] = rate(lambda: C.write_unr(torch, half, unr),
                                                      nbytes // 2)
        for g in (256, 1024, 2048):
            res["write"][f"unr{unr}@{g}"] = rate(lambda: C.write_unr(torch, b, unr, g), nbytes)
        for nt in (0, 1):
            res.setdefault("copy_unr", {})[f"unr{unr}_oneshot{'_nt' if nt else ''}"] = rate(
                lambda: C.copy_unr(torch, a, b, unr, 0, bool(nt)), 2 * nbytes)
    res["copy"] = {}
    for v in range(16):
        nm = ("ntload_" if v & 8 else "") + names[v & 7]
        for g in grids[3:]:
            res["copy"][f"{nm}@{g}"] = rate(lambda: C.copy_var(torch, a, b, g, v), 2 * nbytes)
    # 32 KiB block copies inside the 4 GiB buffer: which side's locality
    # matters (a quarter of the blocks move; sources and destinations
    # disjoint)
    import numpy as np
    blk = 32768
    nblk = nbytes // blk
    npairs = nblk // 4
    rng = np.random.default_rng(3)
    perm = rng.permutation(nblk).astype(np.int32)
    lo = np.arange(npairs, dtype=np.int32)                       # a contiguous run
    hi = np.arange(nblk // 2, nblk // 2 + npairs, dtype=np.int32)
    rs, rd = perm[:npairs], perm[npairs:2 * npairs]              # random, disjoint
    rs_hi = rs[(rs >= npairs)][:npairs // 2]                     # random, outside lo
    patterns = {
        "seq_src_seq_dst": (hi, lo),
        "rand_src_seq_dst": (np.sort(rs_hi), lo[:len(rs_hi)]),
        "rand_unsorted_src_seq_dst": (rs_hi, lo[:len(rs_hi)]),
        "seq_src_rand_dst": (lo[:len(rs_hi)], np.sort(rs_hi)),
        "rand_src_sorted_dst": (rs[np.argsort(rd)], np.sort(rd)),
        "rand_src_rand_dst": (rs, rd),
    }
    res["block_copy"] = {}
    a.fill_(1)
    for name, (src, dst) in patterns.items():
        pd = torch.from_numpy(np.ascontiguousarray(np.stack([src, dst], 1), dtype=np.int32)).to(dev)
        moved = 2 * len(src) * blk
        res["block_copy"][name] = rate(lambda: C.block_copy(torch, a, pd, blk), moved)
        for unr in (1, 2, 4):
            res["block_copy"][f"{name}_piece{4 * unr}k"] = rate(
                lambda: C.block_copy_unr(torch, a, pd, blk, unr), moved)
    # one 16-byte unit a thread, by workgroup size (16 * threads bytes a
    # workgroup): flat write, flat copy, and the two block-copy patterns the
    # relocation plan produces
    res["by_threads"] = {}
    half_a, half_b = a[: a.numel() // 2], b[: b.numel() // 2]
    seq = {k: torch.from_numpy(np.ascontiguousarray(np.stack(patterns[k], 1), dtype=np.int32)).to(dev)
           for k in ("seq_src_seq_dst", "rand_src_seq_dst")}
    for nth in (64, 128, 256, 512):
        r = {"write": rate(lambda: C.write_nth(torch, b, nth), nbytes),
             "copy": rate(lambda: C.copy_nth(torch, half_a, half_b, nth), nbytes)}
        for k, pd in seq.items():
            r[k] = rate(lambda: C.block_copy_nth(torch, a, pd, blk, nth), 2 * pd.shape[0] * blk)
        res["by_threads"][f"{nth}_threads_{16 * nth}B"] = r
    best_w = max(res["write"].items(), key=lambda kv: kv[1])
    best_c = max(res["copy"].items(), key=lambda kv: kv[1])
    return _line("HBM write and copy ceilings: independent writers and store variants (4 GiB)",
                 best_w[1], "GB/s", nbytes / best_w[1] / 1e6, args, "u8",
                 {"workload": "flat 4 GiB writes and 4 GiB -> 4 GiB copies"},
                 best_write=best_w[0], best_copy=best_c[0], best_copy_GBps=best_c[1],
                 results=res)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the path shards by sequence or KV head with no exchange, so the one-GPU "
              "figure is the per-GPU figure)", file=sys.stderr)
        sys.exit(2)
    import torch
    from rustral_amd import kv

    dev = torch.device("cuda:0")
    if args.workload != "config2":
        line = {"config0": run_config0, "config1": run_config1, "config3": run_config3,
                "prefill": run_prefill, "decode_q": run_decode_q,
                "config4": run_config4, "device_step": run_device_step,
                "ceilings": run_ceilings, "store_variants": run_store_variants,
                "patterns_1byte": run_patterns_1byte}[args.workload](
                    torch, dev, args)
        print(json.dumps(line), flush=True)
        return
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
    # the library's pick for this shape (decode_attention asks for it itself)
    part_tokens = kv.partition_size_for(B, HQ, HKV, D, kv.RKV_BF16, max_ctx)
    part_waves = 4 if part_tokens <= 640 else 8

    def call(i, passes, workspace=None):
        q, k, v, t = layers[i]
        kv.decode_attention(q, k, v, t, ctx_d, scale, max_context=max_ctx, out=outs[i],
                            workspace=ws if workspace is None else workspace, passes=passes)

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(args.warmup):
            for i in range(n_layers):
                call(i, "both")
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    # (1) value: the step as a serving loop runs it -- the 32 calls (both
    # passes each) captured once in a HIP graph; K steps = K replays.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(n_layers):
            call(i, "both")
    graph.replay()
    # untimed replays for at least 100 ms more: the clock takes ~15 ms of
    # sustained load to settle
    warm_replays, t_warm = 1, time.perf_counter()
    while time.perf_counter() - t_warm < 0.1:
        for _ in range(4):
            graph.replay()
        torch.cuda.synchronize()
        warm_replays += 4
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    start, stop = ev(), ev()
    marks_step = [ev() for _ in range(args.steps + 1)]   # per-replay boundaries
    torch.cuda.synchronize()
    start.record()
    marks_step[0].record()
    for s in range(args.steps):
        graph.replay()
        marks_step[s + 1].record()
    stop.record()
    torch.cuda.synchronize()
    ms_step = start.elapsed_time(stop) / args.steps
    step_stats = stats([marks_step[i].elapsed_time(marks_step[i + 1]) for i in range(args.steps)])
    del graph

    # (2) roofline: the partition kernel alone, HIP events on its launch
    # stream around bursts of the n_layers partition launches issued back to
    # back (each layer with a workspace of its own; the merges follow each
    # burst): a launch's share is the kernel's duration plus the gap to the
    # next launch.
    ws_layer = [torch.empty_like(ws) for _ in range(n_layers)]
    bursts = [(ev(), ev()) for _ in range(args.steps)]
    torch.cuda.synchronize()
    for s in range(args.steps):
        bursts[s][0].record()
        for i in range(n_layers):
            call(i, "partitions", ws_layer[i])
        bursts[s][1].record()
        for i in range(n_layers):
            call(i, "merge", ws_layer[i])
    torch.cuda.synchronize()
    avg_burst_part_us = 1e3 * sum(a.elapsed_time(b) for a, b in bursts) / (args.steps * n_layers)
    del ws_layer

    # (3) the same steps launched eagerly with events around every partition
    # and merge launch (each launch's figure then includes its dispatch).
    marks = [[(ev(), ev(), ev()) for _ in range(n_layers)] for _ in range(args.steps)]
    e0, e1 = ev(), ev()
    torch.cuda.synchronize()
    e0.record()
    for s in range(args.steps):
        for i in range(n_layers):
            a, m, e = marks[s][i]
            a.record()
            call(i, "partitions")
            m.record()
            call(i, "merge")
            e.record()
    e1.record()
    torch.cuda.synchronize()
    ms_step_eager = e0.elapsed_time(e1) / args.steps
    part_ms = [a.elapsed_time(m) for row in marks for (a, m, e) in row]
    merge_ms = [m.elapsed_time(e) for row in marks for (a, m, e) in row]
    avg_part_us = 1e3 * sum(part_ms) / len(part_ms)
    avg_merge_us = 1e3 * sum(merge_ms) / len(merge_ms)
    bytes_call = algorithmic_bytes(ctx)
    call_us = 1e3 * ms_step / n_layers
    value = bytes_call / (call_us * 1e-6) / 1e9
    achieved = bytes_call / (avg_burst_part_us * 1e-6) / 1e9
    tokens_per_s = B / (ms_step * 1e-3) * (n_layers / 32)

    traffic = traffic_from_profiles()
    copy_gbps = copy_bandwidth(torch, dev)
    read_gbps = read_bandwidth(torch, dev)
    cpu = None
    if not args.no_cpu_baseline:
        # 16 threads: the host share of one GPU on the box (nproc there counts
        # the whole host); the host's nproc and CPU model are recorded beside
        threads = args.cpu_threads or min(os.cpu_count() or 1, 16)
        cpu = cpu_baseline(torch, layers, ctx, threads)
        m = machine(torch)
        cpu.update({"cpu_model": m["cpu_model"], "host_nproc": m["host_nproc"],
                    "host_cpus_usable": m["host_cpus_usable"],
                    "threads_note": "threads = min(nproc, 16): the CPU share of one GPU on the box"})

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
                   "layers_per_step": n_layers,
                   "step": "one decode token: 32 attention calls, replayed from a HIP graph"},
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBPS, 2),
        "decode_tokens_per_s_b64": round(tokens_per_s, 1),
        "us_per_call": round(call_us, 2),
        "step_ms_stats": step_stats,
        "untimed_replays_before_timing": warm_replays,
        "value_at_p50_step": round(bytes_call * n_layers / (step_stats["p50"] * 1e-3) / 1e9, 2),
        "step_ms_eager_with_events": round(ms_step_eager, 4),
        "partition_kernel_us": round(avg_burst_part_us, 2),
        "partition_kernel_us_events_per_launch": round(avg_part_us, 2),
        "merge_kernel_us": round(avg_merge_us, 2),
        "algorithmic_bytes_per_call": bytes_call,
        "measured_copy_GBps": round(copy_gbps, 1),
        "measured_read_GBps": None if read_gbps is None else round(read_gbps, 1),
        "value_over_measured_read": None if read_gbps is None else round(value / read_gbps, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "kernel": (f"decode_stream_kernel<bf16, D=128, G=4> ({part_tokens}-token "
                                f"partitions, {part_waves} waves each, K/V tiles staged in LDS, "
                                "MFMA QK^T and PV)"),
                     "traffic": traffic},
        "cpu_baseline": cpu,
        "machine": machine(torch),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
