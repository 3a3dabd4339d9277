"""Builds libmk.so (the HIP kernels + C ABI) in-tree for gfx950 with hipcc.

    python -m minicpm5_mk._build          # from minicpm5-vllm-tpu_amd/

Every source under ../csrc is compiled with `hipcc --offload-arch=gfx950 -O3` (packed-FP32
instructions disabled) into an object file under ../_build/, then linked into
minicpm5_mk/libmk.so next to this file.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
PROJ = os.path.dirname(PKG)
ROOT = os.path.dirname(PROJ)
CSRC = os.path.join(PROJ, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(PROJ, "_build")
LIB = os.path.join(PKG, "libmk.so")
ARCH = "gfx950"

SOURCES = ["api.cpp", "model.cpp", "attn.hip", "gemm.hip", "norm.hip", "pack.hip", "peak.hip", "noalloc.hip", "prep.hip"]
# attention scores are finite or -inf, never NaN: without NaN semantics the row max needs no
# canonicalising v_max per MFMA result
EXTRA = {"attn.hip": ["-fno-honor-nans"]}
CFLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
          "-packed-fp32-ops", "-Wno-unused-result", f"-I{INCLUDE}", f"-I{CSRC}"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libmk)")


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *CFLAGS, *EXTRA.get(src, []), "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compiles every source and links libmk.so; returns its path.  Always rebuilds."""
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
