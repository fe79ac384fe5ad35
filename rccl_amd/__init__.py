"""rccl_amd: MI355X-native ordering primitives (radix sort, merge, merge sort,
set operations) with the reference's CUB/Thrust-style host surface.

The compute path is ``librccl_hip.so`` (hand-written gfx950 HIP kernels behind
the C ABI in ``include/rccl_hip.h``). Import ``rccl_amd.cub`` or
``rccl_amd.thrust`` for the host mirror; both need a GPU and the built
library and raise when either is missing.
"""
from ._abi import LIB_PATH, DeviceAlgorithmError, load  # noqa: F401

__all__ = ["LIB_PATH", "DeviceAlgorithmError", "load"]
