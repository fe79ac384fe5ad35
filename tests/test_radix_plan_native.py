"""The radix sort's host-side planning logic under sanitizers, on the CPU.

tests/native/radix_plan_check.cpp includes the library's own plan and layout
header (rccl_amd/csrc/radix_plan.hpp, plain C++) and is built with g++ under
AddressSanitizer and UndefinedBehaviorSanitizer. It checks:
- assign_plan for P = 4 and 8 passes (the merge-sort lowering) and 4N (the
  record sort's N-word rows): every trivial-pass mask up to 16 passes (then
  structured and random masks) under each of the four plan-flag
  combinations. The first active pass reads the input, each later one what
  the previous wrote, the last writes the output; no pass reads and writes
  one buffer (an in-place stream's input and output are one); look-back
  buffers and conversion flags alternate as the kernels expect; simulating
  the data flow of an in-place and a copied stream, the output holds every
  non-trivial pass in order.
- layout near 2^30 and 2^32 - 1 items, recomputed in 128-bit arithmetic:
  aligned, disjoint regions sized for the tiles and groups, 64-bit look-back
  descriptors from 2^30 items.
The reference gates the same path with compute-sanitizer memcheck and
racecheck over its probes (scripts/test-ordering-results.sh:50-65); GPU
sanitizers are not available here, so the host logic is checked this way.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_radix_plan_and_layout_under_sanitizers(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not installed")
    exe = tmp_path / "radix_plan_check"
    build = subprocess.run(
        [gxx, "-std=c++17", "-O1", "-g", "-Wall", "-Werror", "-fsanitize=address,undefined",
         "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
         "-I", os.path.join(ROOT, "rccl_amd", "csrc"),
         os.path.join(ROOT, "tests", "native", "radix_plan_check.cpp"), "-o", str(exe)],
        capture_output=True, text=True, timeout=300)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "all radix plan and layout checks passed" in run.stdout
