"""Builds librustral_kv.so (HIP kernels + C ABI) for gfx950 with hipcc.

Usage: ``python -m rustral_amd.build`` (also called by ``__graft_entry__.build``).
Objects go to ``rustral_amd/_build/``, the library to ``rustral_amd/lib/``; both
stay in-tree so the built library travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "librustral_kv.so")
ARCH = os.environ.get("RKV_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # packed fp32 ops stay off (v_pk_* fp32 forms are not trusted on this pool)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: cannot build librustral_kv.so")


# host-only C++ (block manager, scheduler): plain g++, no device code
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra"]


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC)
                  if f.endswith(".hip") or f.endswith(".cpp"))


def _obj(src: str) -> str:
    return os.path.join(OBJ_DIR, os.path.basename(src) + ".o")


def _stale(src: str) -> bool:
    """True if src (or a header it may include) is newer than its object."""
    obj = _obj(src)
    if not os.path.exists(obj):
        return True
    deps = [src, os.path.join(CSRC, "common.hpp"), *[
        os.path.join(HERE, "..", "include", h) for h in os.listdir(os.path.join(HERE, "..", "include"))]]
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(d) > t for d in deps if os.path.exists(d))


def _compile(src: str) -> str:
    obj = _obj(src)
    if src.endswith(".cpp"):
        cmd = [os.environ.get("CXX", "g++"), *CXX_FLAGS, "-c", src, "-o", obj]
    else:
        cmd = [hipcc(), *HIPCC_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


CEILING_SRC = os.path.join(HERE, "ceiling", "ceiling.hip")
CEILING_LIB = os.path.join(LIB_DIR, "librkv_ceiling.so")


def build_ceiling(verbose: bool = False) -> str:
    """The measurement library of bench.py's ceilings workload (stream
    kernels, not part of librustral_kv.so)."""
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = CEILING_LIB + ".tmp"
    r = subprocess.run([hipcc(), *HIPCC_FLAGS, "-shared", "-o", tmp, CEILING_SRC],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed for {CEILING_SRC}:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, CEILING_LIB)
    if verbose:
        print(f"built {CEILING_LIB}", file=sys.stderr)
    return CEILING_LIB


def build(verbose: bool = False, changed_only: bool = False) -> str:
    """Compiles every source (or, with changed_only, those newer than their
    objects) and links the library."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sources()
    todo = [s for s in srcs if _stale(s)] if changed_only else srcs
    with cf.ThreadPoolExecutor(max_workers=max(1, min(8, len(todo)))) as ex:
        list(ex.map(_compile, todo))
    objs = [_obj(s) for s in srcs]
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}", file=sys.stderr)
    if not changed_only or not os.path.exists(CEILING_LIB) or \
            os.path.getmtime(CEILING_SRC) > os.path.getmtime(CEILING_LIB):
        build_ceiling(verbose)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True, changed_only="--changed" in sys.argv[1:])
