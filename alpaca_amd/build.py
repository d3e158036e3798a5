"""Builds libalpaca_hip.so in-tree with hipcc for gfx950.

Usage: python -m alpaca_amd.build [-j N] [--incremental]
Each source compiles to an object under alpaca_amd/_build/ in parallel, then
the objects link into alpaca_amd/libalpaca_hip.so.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libalpaca_hip.so")
# (source, object name, extra defines).  kernels_decode.hip is compiled once per
# (weight format, head dim) variant of the persistent decode kernel, so the
# large inlined kernels build in parallel, and once for its host side.
DECODE_VARIANTS = [(fmt, hd) for fmt in ("q8", "q4", "f16") for hd in (64, 128)]
DECODE_FMT_ENUM = {"q8": "DT_Q8_0", "q4": "DT_Q4_0", "f16": "DT_F16"}
SOURCES = [("kernels_decode.hip", f"kernels_decode_{fmt}_hd{hd}",
            [f"-DDECODE_FMT={DECODE_FMT_ENUM[fmt]}", f"-DDECODE_HD={hd}", f"-DDECODE_ENTRY=decode_kernel_{fmt}_hd{hd}"])
           for fmt, hd in DECODE_VARIANTS]
SOURCES += [(src, os.path.splitext(src)[0], []) for src in
            ("kernels_decode.hip", "kernels_misc.hip", "kernels_gemv.hip", "kernels_sample.hip", "runtime.cpp",
             "gguf.cpp", "shim.cpp", "noalloc.cpp")]
# The prefill GEMMs scale each MFMA result on the VALU, and flash attention
# rescales its output accumulators every key block; the VGPR form of the MFMA
# keeps those results where the VALU reads them (the AGPR form adds a
# v_accvgpr_read / write per result register).
SOURCES += [(src, os.path.splitext(src)[0], ["-mllvm", "-amdgpu-mfma-vgpr-form=1"])
            for src in ("kernels_gemm.hip", "kernels_attention.hip")]
ARCH = "gfx950"
# Packed FP32 instructions are disabled: hipcc -O3 otherwise emits v_pk_* forms.
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _stale(src: str, obj: str) -> bool:
    """An object is stale when it is older than its source or any header in csrc/."""
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = [os.path.join(CSRC, src)] + [os.path.join(CSRC, h) for h in os.listdir(CSRC) if h.endswith(".h")]
    return any(os.path.getmtime(d) > t for d in deps)


def _compile(item, incremental: bool = False) -> str:
    src, name, defines = item
    obj = os.path.join(BUILD, name + ".o")
    if incremental and not _stale(src, obj):
        return obj
    cmd = [hipcc(), *FLAGS, *defines, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


# A stand-alone gfx950 code object for the shim's module-load tests.
SHIM_SRC, SHIM_CO = "shim_kernels.hip", os.path.join(HERE, "shim_kernels.hsaco")


def _code_object() -> str:
    cmd = [hipcc(), "-O3", "-std=c++17", f"--offload-arch={ARCH}", "--genco", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", os.path.join(CSRC, SHIM_SRC), "-o", SHIM_CO + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"code object build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(SHIM_CO + ".tmp", SHIM_CO)
    return SHIM_CO


def build(jobs: int = 0, incremental: bool = False) -> str:
    """Compiles every source (incremental: only objects older than their
    source or a csrc/ header) and links the library."""
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        co = None
        if not (incremental and os.path.exists(SHIM_CO) and
                os.path.getmtime(SHIM_CO) > os.path.getmtime(os.path.join(CSRC, SHIM_SRC))):
            co = ex.submit(_code_object)
        objs = list(ex.map(lambda it: _compile(it, incremental), SOURCES))
        if co:
            co.result()
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=0)
    ap.add_argument("--incremental", action="store_true", help="recompile only stale objects")
    a = ap.parse_args()
    print(build(a.j, a.incremental))
    sys.exit(0)
