"""Rules for the machine code of libmk.so, checked on its disassembly (CPU only, code built here).

Every gfx950 code object in the built library is unbundled into a scratch directory and disassembled
with ROCm's llvm-objdump, and the instruction stream is checked for two classes this build keeps out of
its GPU code:

* writes through the scalar data cache -- scalar stores, scalar atomics, and that cache's write-back
  and discard: device memory is written only with vector stores and vector atomics (the attention's
  work-queue counters, the QKV epilogue's queue reset);
* packed FP32 arithmetic: the sources are compiled with the packed-fp32-ops target feature off, so no
  such instruction is generated and none is written by hand.

Skipped when the library has not been built or the ROCm tools are missing.
"""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "minicpm5-vllm-tpu_amd", "minicpm5_mk", "libmk.so")
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"

SCALAR_WRITES = re.compile(r"\bs_(store|buffer_store|scratch_store|atomic|buffer_atomic|dcache_wb|dcache_discard)\w*")
PACKED_F32 = re.compile(r"\bv_pk_(add|mul|fma)_f32\b")


def _disassembly():
    if not os.path.exists(LIB) or not os.path.exists(OBJDUMP):
        pytest.skip("libmk.so or llvm-objdump not present")
    with tempfile.TemporaryDirectory() as d:
        lib = os.path.join(d, "libmk.so")
        shutil.copy(LIB, lib)
        subprocess.run([OBJDUMP, "--offloading", lib], cwd=d, check=True, capture_output=True, timeout=120)
        objs = sorted(f for f in os.listdir(d) if "amdgcn" in f and "gfx950" in f)
        assert objs, "no gfx950 code object in libmk.so"
        out = {}
        for f in objs:
            r = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", os.path.join(d, f)], check=True,
                               capture_output=True, text=True, timeout=300)
            out[f] = r.stdout
        return out


def test_device_code_rules():
    dis = _disassembly()
    assert sum(len(t) for t in dis.values()) > 100000, "disassembly unexpectedly small"
    assert any("v_mfma" in t for t in dis.values()), "no MFMA instruction found: wrong code object?"
    bad = {}
    for f, text in dis.items():
        hits = sorted(set(m.group(0) for m in SCALAR_WRITES.finditer(text)))
        hits += sorted(set(m.group(0) for m in PACKED_F32.finditer(text)))
        if hits:
            bad[f] = hits
    assert not bad, bad
