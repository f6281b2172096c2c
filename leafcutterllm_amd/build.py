"""Build recipe for the product library leafcutterllm_amd/liblcmoe.so.

hipcc compiles the HIP translation units for gfx950 only; g++ compiles the
host-only sources (utilities and the GGUF reader).  Every build compiles from source (no caching), so a
call always reflects the current sources.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
ROOT = os.path.dirname(PKG)
BUILD = os.path.join(ROOT, "_build")
LIB = os.path.join(PKG, "liblcmoe.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # every fused multiply-add is explicit (__builtin_fmaf); nothing else fuses
    "-ffp-contract=off",
    # no packed-FP32 instructions (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-flush-denormals-to-zero",
    "-Wall", "-Wno-unused-function",
]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-pthread", "-Wall",
              "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    jobs = []
    for src in sorted(os.listdir(CSRC)):
        if src.endswith(".hip"):
            o = os.path.join(BUILD, src[:-4] + ".o")
            jobs.append(([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", o], o))
    for src in sorted(os.listdir(CSRC)):
        if src.endswith(".cpp"):
            o = os.path.join(BUILD, src[:-4] + ".o")
            jobs.append((["g++", *HOST_FLAGS, "-c", os.path.join(CSRC, src), "-o", o], o))
    # one compiler per source, at most MAX_JOBS (or the CPU count) at once
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", 0)) or os.cpu_count() or 1, 16))
    with ThreadPoolExecutor(workers) as pool:
        for f in [pool.submit(_run, cmd, verbose) for cmd, _ in jobs]:
            f.result()
    objs = [o for _, o in jobs]
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-pthread", *objs, "-o", tmp],
         verbose)
    shutil.move(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
