"""Build bench_probes/libscatter_probe.so (gfx950), the memory-pattern probe
that bench.py's hbm_reference leg times beside torch's copy and read."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "scatter_probe.hip")
LIB_PATH = os.path.join(HERE, "libscatter_probe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-Wall",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def build() -> str:
    """Compile the probe. Always recompiles."""
    tmp = LIB_PATH + ".tmp"
    res = subprocess.run([HIPCC, *FLAGS, SRC, "-o", tmp], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {SRC}:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build())
