"""Build the gfx950 HIP library in-tree: funasrnet_amd/libfunasr_hip.so.

hipcc cross-compiles for gfx950 without a GPU. Flags: no FMA contraction
(-ffp-contract=off) because the kernels restate the reference's float order,
fp32 denormals kept, and packed-fp32 instruction selection disabled.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIBRARY = os.path.join(HERE, "libfunasr_hip.so")
# Host-only helper of the benchmark: native worker threads that step the
# batcher (no HIP code; built with the host compiler).
BENCH_WORKERS = os.path.join(HERE, "libfah_bench_workers.so")
SOURCES = ["fah_kernels.hip", "fah_persistent.hip", "fah_prefill.hip", "fah_sessions.hip", "fah_float.hip",
           "fah_api.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-fno-gpu-flush-denormals-to-zero", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         # MFMA results in VGPRs: the fp32 epilogue reads them without accvgpr copies.
         "-mllvm", "-amdgpu-mfma-vgpr-form",
         "-Wall", "-Wno-unused-function"]


def _compile(source: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(source)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(SRC, source), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source}:\n{r.stderr}")
    return obj


def build() -> str:
    """Compile every source and link the shared library (always rebuilds)."""
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        objects = list(pool.map(_compile, SOURCES))
    tmp = LIBRARY + ".tmp"
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objects, "-o", tmp],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIBRARY)
    r = subprocess.run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-pthread", os.path.join(SRC, "bench_workers.cpp"),
                        "-o", BENCH_WORKERS], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"bench_workers.cpp failed:\n{r.stderr}")
    return LIBRARY


if __name__ == "__main__":
    print(build())
    sys.exit(0)
