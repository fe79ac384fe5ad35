"""Build librccl_hip.so (gfx950 HIP kernels + C ABI) in-tree with hipcc.

The shared library is written to ``rccl_amd/librccl_hip.so``; object files go
to ``rccl_amd/_build/``. Sources compile in parallel, one hipcc per file.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_PATH = os.path.join(HERE, "librccl_hip.so")
INCLUDE = os.path.join(ROOT, "include")

SOURCES = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# gfx950 only. Packed FP32 instructions are disabled for all device code.
# The atomic optimizer is off: it rewrites single-lane atomics into a
# wave-wide sequence that consumes the returned value at once, which turns
# the onesweep's early tile claim into a full memory-counter wait.
COMPILE_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-fvisibility=hidden",
    "-I" + INCLUDE,
    "-I" + CSRC,
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMPILE_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> str:
    """Compile every source and link librccl_hip.so. Always recompiles."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
