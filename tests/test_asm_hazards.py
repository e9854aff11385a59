"""CPU check of the generated gfx950 code: no instruction other than an MFMA
touches an MFMA's destination registers within 8 wait states on any path.
Every source that issues MFMAs is compiled to assembly (device code only)
with the library's own flags."""
import concurrent.futures as cf
import os
import subprocess
import tempfile

import pytest

from rustral_amd import build as B
from tests.asm_hazards import analyse, scan

CSRC = B.CSRC
MFMA_SOURCES = sorted(f for f in os.listdir(CSRC)
                      if f.endswith(".hip") and "mfma" in open(os.path.join(CSRC, f)).read())


def test_scanner_finds_a_planted_read():
    """The scanner itself: a VALU read two instructions after an MFMA, and the
    same read reached through a branch, are findings; one 8 wait states
    later (s_nop 7 covers 8) is not."""
    near = ["\tv_mfma_f32_16x16x32_bf16 v[10:13], v[2:5], v[6:9], 0",
            "\tv_mov_b32_e32 v1, v0",
            "\tv_add_f32_e32 v20, v11, v1"]
    assert len(analyse(near)) == 1
    branch = ["\tv_mfma_f32_16x16x32_bf16 a[0:3], v[2:5], v[6:9], 0",
              "\ts_cbranch_scc1 .LBB0_2",
              "\ts_nop 7",
              "\ts_nop 7",
              ".LBB0_2:",
              "\tv_accvgpr_read_b32 v1, a2"]
    assert len(analyse(branch)) == 1
    far = ["\tv_mfma_f32_16x16x32_bf16 v[10:13], v[2:5], v[6:9], 0",
           "\ts_nop 7",
           "\tv_add_f32_e32 v20, v11, v1"]
    assert analyse(far) == []


def _asm(src: str, out_dir: str) -> str:
    out = os.path.join(out_dir, os.path.basename(src) + ".s")
    cmd = [B.hipcc(), *[f for f in B.HIPCC_FLAGS if f not in ("-fPIC", "-Wall")],
           "--cuda-device-only", "-S", src, "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {src}:\n{r.stderr[-2000:]}")
    return out


@pytest.mark.timeout(600)
def test_generated_code_has_no_early_mfma_result_access():
    try:
        B.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    assert MFMA_SOURCES, "expected MFMA-using sources"
    with tempfile.TemporaryDirectory() as tmp, cf.ThreadPoolExecutor(len(MFMA_SOURCES)) as ex:
        paths = list(ex.map(lambda f: _asm(os.path.join(CSRC, f), tmp), MFMA_SOURCES))
        findings = []
        for p in paths:
            text = open(p).read()
            assert "v_mfma" in text, p
            findings += [(os.path.basename(p), *f) for f in scan(text)]
    assert not findings, "\n".join(f"{f}: {n[:60]}: {d} wait states: {m[:48]} -> {u[:48]}"
                                   for f, n, d, m, u in findings[:10])
