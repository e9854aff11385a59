"""The safetensors reader under AddressSanitizer and UndefinedBehaviorSanitizer
(host code, CPU): tests/fuzz/safetensors_fuzz.cpp mutates a valid decoder
file thousands of times and runs every mutation through the reader and the
strict loader; any out-of-bounds access, leak or undefined behaviour aborts
the run."""
import os
import shutil
import subprocess

import pytest

from rustral_amd import model

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.timeout(600)
def test_reader_survives_mutated_files_under_sanitizers(tmp_path):
    cxx = shutil.which("g++")
    if not cxx:
        pytest.skip("g++ not available")
    exe = tmp_path / "st_fuzz"
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]
    cmd = [cxx, "-std=c++17", "-O1", "-g", *san, "-o", str(exe),
           os.path.join(ROOT, "tests", "fuzz", "safetensors_fuzz.cpp"),
           os.path.join(ROOT, "rustral_amd", "csrc", "safetensors.cpp")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    cfg = model.config(vocab=50, d_model=64, n_heads=4, n_kv_heads=2, d_ff=96, n_layers=2,
                       max_seq=32)
    seed = tmp_path / "good.safetensors"
    model.save_safetensors(cfg, model.init_params(cfg, seed=1, std=0.5), seed)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([str(exe), str(seed), str(tmp_path / "mut.safetensors"), "20000"],
                       capture_output=True, text=True, env=env, timeout=500)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    acc, rej = (int(x) for x in r.stdout.split()[1::2])
    assert acc > 0 and rej > 0 and acc + rej == 20000
