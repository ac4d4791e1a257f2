"""Build libswiftrwkv_hip.so in-tree: HIP kernels for gfx950 + host C++.

Run as `python -m swiftrwkv_amd.build` (or through __graft_entry__.build()).
Cross-compiles without a GPU.  Object files go to swiftrwkv_amd/_build/.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libswiftrwkv_hip.so")
ARCH = os.environ.get("SWIFTRWKV_ARCH", "gfx950")

HIP_SOURCES = ["wkv7.hip", "wkv7_chunked.hip", "rwkvq.hip", "x070.hip", "gemm.hip", "gemv_mfma.hip", "prefill.hip"]
HOST_SOURCES = ["host.cpp", "manifest.cpp"]

# Packed-FP32 VALU ops are disabled for every device compile.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-ffp-contract=fast",
    # code object v5: loadable by the HIP 7.0 runtime torch bundles and by ROCm 7.2
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

# The batched matrix-core GEMV reads every MFMA result with VALU ops: results
# in VGPRs (not AGPRs) save a v_accvgpr_read per result dword.
FILE_FLAGS = {"gemv_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP extension cannot be built")


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({' '.join(cmd)}):\n{r.stdout}")
    return r.stdout


def build(verbose: bool = False, extra_hip_flags=()) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = _hipcc()
    jobs = []
    objs = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        objs.append(obj)
        jobs.append([hipcc, *HIP_FLAGS, *FILE_FLAGS.get(src, ()), *extra_hip_flags, "-c", os.path.join(CSRC, src),
                     "-o", obj])
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD, src.replace(".cpp", ".o"))
        objs.append(obj)
        jobs.append(["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-c", os.path.join(CSRC, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        outs = list(ex.map(_run, jobs))
    if verbose:
        for o in outs:
            if o.strip():
                print(o)
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-lpthread"])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
