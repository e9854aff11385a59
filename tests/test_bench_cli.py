"""bench.py's contract pieces that run without a GPU: the multi-GPU request
is refused with a message before anything touches a device, and the
roofline's algorithmic byte count (the numerator of `roofline.achieved`)
is the count of what one decode call must move."""
import os
import subprocess
import sys

import numpy as np

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT,
                       env={**os.environ, "HIP_VISIBLE_DEVICES": ""})
    assert r.returncode == 2
    assert "--gpus 2 is not supported" in r.stderr
    assert r.stdout == ""


def test_algorithmic_bytes_known_answer():
    # contexts 1, 16 and 17 tokens at Hkv 8, D 128, bf16 K and V:
    #   K + V rows: 34 tokens x 8 heads x 128 dims x 2 B x 2      = 139,264
    #   q read + out written, fp32: 3 x 32 heads x 128 x 4 B x 2 =  98,304
    #   block ids 1 + 1 + 2 and three lengths, 4 B each          =      28
    assert bench.algorithmic_bytes(np.array([1, 16, 17])) == 139_264 + 98_304 + 28


def test_algorithmic_bytes_of_the_headline_workload():
    # the per-call figure the profiles divide by the kernel time
    ctx = np.random.default_rng(bench.SEED).integers(bench.CTX_LO, bench.CTX_HI + 1, size=bench.B)
    assert bench.algorithmic_bytes(ctx) == 635_705_484
    blocks = int(((ctx + bench.BS - 1) // bench.BS).sum())
    kv = int(ctx.sum()) * bench.HKV * bench.D * 2 * 2
    assert bench.algorithmic_bytes(ctx) - kv == (bench.B * bench.HQ * bench.D * 8
                                                  + 4 * blocks + 4 * bench.B)
