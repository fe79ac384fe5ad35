"""ctypes binding of the rccl_hip C ABI (include/rccl_hip.h).

The library is ``rccl_amd/librccl_hip.so`` built in-tree by
``rccl_amd.build``. Loading fails loudly when it is missing: there is no CPU
or PyTorch fallback for any operation.

When PyTorch is importable it is imported before the library is loaded, so a
process that also uses PyTorch for device memory runs a single HIP runtime.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# The in-tree build; RCCL_HIP_LIBRARY may name another build of the same
# library (for example one compiled with different tuning macros).
LIB_PATH = os.environ.get("RCCL_HIP_LIBRARY") or os.path.join(HERE, "librccl_hip.so")

# Enumerations (values equal include/rccl_hip.h).
SUCCESS = 0
STATUS_NAMES = {
    0: "Success",
    1: "LengthMismatch",
    2: "WorkspaceTooSmall",
    3: "InvalidBitRange",
    4: "UnsupportedTarget",
    5: "SizeOverflow",
    6: "Memory",
    7: "Driver",
    8: "Launch",
    9: "InvalidArgument",
}
KEY_KINDS = {
    "u32": 0, "i32": 1, "f32": 2, "u64": 3, "i64": 4, "f64": 5,
    "u8": 6, "i8": 7, "u16": 8, "i16": 9,
}
RADIX_KINDS = ("u32", "i32", "f32", "u64", "i64", "f64")
ASCENDING = 0
DESCENDING = 1
RANKING = {"auto": 0, "lane_atomic": 1, "match_any": 2}
TILE_ORDER = {"auto": 0, "ticket": 1}
SET_OPS = {"union": 0, "intersection": 1, "difference": 2, "symmetric_difference": 3}
GROUP_UNIQUE = 0
GROUP_OPS = {"natural_bag_add": 1, "boolean_or": 2, "independent_probability_or": 3}

# The exported C symbols; a test checks the library exports each one.
EXPORTED_SYMBOLS = (
    "rccl_hip_last_error",
    "rccl_hip_status_string",
    "rccl_hip_abi_version",
    "rccl_hip_program_load",
    "rccl_hip_timing_enable",
    "rccl_hip_timing_read",
    "rccl_hip_radix_sort_workspace_bytes",
    "rccl_hip_radix_sort_buffer",
    "rccl_hip_radix_sort",
    "rccl_hip_radix_sort_static",
    "rccl_hip_radix_configure",
    "rccl_hip_merge_workspace_bytes",
    "rccl_hip_merge",
    "rccl_hip_merge_sort_workspace_bytes",
    "rccl_hip_merge_sort",
    "rccl_hip_set_op_workspace_bytes",
    "rccl_hip_set_op",
    "rccl_hip_set_op_arithmetic",
    "rccl_hip_record_sort_workspace_bytes",
    "rccl_hip_record_sort",
    "rccl_hip_group_workspace_bytes",
    "rccl_hip_unique_copy",
    "rccl_hip_reduce_by_key",
    "rccl_hip_bound_search",
    "rccl_hip_bound_search_workspace_bytes",
)


class ErrorInfo(ctypes.Structure):
    _fields_ = [
        ("status", ctypes.c_int),
        ("role", ctypes.c_char_p),
        ("expected", ctypes.c_uint64),
        ("actual", ctypes.c_uint64),
        ("begin_bit", ctypes.c_uint32),
        ("end_bit", ctypes.c_uint32),
        ("key_bits", ctypes.c_uint32),
        ("hip_error", ctypes.c_int),
    ]


class KernelTiming(ctypes.Structure):
    _fields_ = [
        ("kernel", ctypes.c_char_p),
        ("ms", ctypes.c_float),
        ("items", ctypes.c_uint64),
    ]


class DeviceAlgorithmError(RuntimeError):
    """Mirror of rccl_cub::DeviceAlgorithmError (rccl-cub/src/error.rs:3-25)."""

    def __init__(self, status: int, info: ErrorInfo | None = None):
        self.status = status
        self.kind = STATUS_NAMES.get(status, f"Unknown({status})")
        self.role = info.role.decode() if info is not None and info.role else ""
        self.expected = info.expected if info is not None else 0
        self.actual = info.actual if info is not None else 0
        self.begin = info.begin_bit if info is not None else 0
        self.end = info.end_bit if info is not None else 0
        self.key_bits = info.key_bits if info is not None else 0
        self.hip_error = info.hip_error if info is not None else 0
        super().__init__(self._message())

    def _message(self) -> str:
        if self.kind == "LengthMismatch":
            return f"{self.role} length {self.actual} does not match required length {self.expected}"
        if self.kind == "WorkspaceTooSmall":
            return f"{self.role} length {self.actual} is smaller than required length {self.expected}"
        if self.kind == "InvalidBitRange":
            return (f"radix bit range {self.begin}..{self.end} is outside 0..={self.key_bits} "
                    f"or reversed")
        if self.kind in ("Driver", "Launch", "Memory"):
            return f"{self.kind}: {self.role} (hipError {self.hip_error})"
        return f"{self.kind}: {self.role}"


_lib = None


class _Optional:
    """Declaration target for a symbol the loaded build does not export."""

    def __setattr__(self, name, value):
        pass


def _declare(lib):
    c = ctypes

    class _View:
        def __getattr__(self, name):
            return getattr(lib, name) if hasattr(lib, name) else _Optional()

    lib_view = _View()
    vp, sz, st = c.c_void_p, c.c_size_t, c.c_int
    lib_view.rccl_hip_last_error.restype = None
    lib_view.rccl_hip_last_error.argtypes = [c.POINTER(ErrorInfo)]
    lib_view.rccl_hip_status_string.restype = c.c_char_p
    lib_view.rccl_hip_status_string.argtypes = [st]
    lib_view.rccl_hip_abi_version.restype = c.c_int
    lib_view.rccl_hip_abi_version.argtypes = []
    lib_view.rccl_hip_program_load.restype = st
    lib_view.rccl_hip_program_load.argtypes = [c.c_int]
    lib_view.rccl_hip_timing_enable.restype = st
    lib_view.rccl_hip_timing_enable.argtypes = [c.c_int]
    lib_view.rccl_hip_timing_read.restype = st
    lib_view.rccl_hip_timing_read.argtypes = [c.POINTER(KernelTiming), sz, c.POINTER(sz)]
    lib_view.rccl_hip_radix_sort_workspace_bytes.restype = st
    lib_view.rccl_hip_radix_sort_workspace_bytes.argtypes = [st, sz, sz, c.POINTER(sz)]
    lib_view.rccl_hip_radix_sort_buffer.restype = st
    lib_view.rccl_hip_radix_sort_buffer.argtypes = [st, sz, st, vp, vp, vp, vp, sz, c.POINTER(c.c_int),
                                               c.c_uint32, c.c_uint32, vp, sz, vp]
    lib_view.rccl_hip_radix_sort.restype = st
    lib_view.rccl_hip_radix_sort.argtypes = [st, sz, st, vp, vp, vp, vp, sz, vp, sz, vp]
    lib_view.rccl_hip_radix_configure.restype = st
    lib_view.rccl_hip_radix_configure.argtypes = [c.c_int, c.c_int]
    lib_view.rccl_hip_radix_sort_static.restype = st
    lib_view.rccl_hip_radix_sort_static.argtypes = [st, sz, st, vp, vp, vp, vp, sz, vp]
    lib_view.rccl_hip_merge_workspace_bytes.restype = st
    lib_view.rccl_hip_merge_workspace_bytes.argtypes = [st, sz, sz, sz, c.POINTER(sz)]
    lib_view.rccl_hip_merge.restype = st
    lib_view.rccl_hip_merge.argtypes = [st, sz, st, vp, vp, sz, vp, vp, sz, vp, vp, vp, sz, vp]
    lib_view.rccl_hip_merge_sort_workspace_bytes.restype = st
    lib_view.rccl_hip_merge_sort_workspace_bytes.argtypes = [st, sz, sz, c.POINTER(sz)]
    lib_view.rccl_hip_merge_sort.restype = st
    lib_view.rccl_hip_merge_sort.argtypes = [st, sz, st, vp, vp, vp, vp, sz, vp, sz, vp]
    lib_view.rccl_hip_record_sort_workspace_bytes.restype = st
    lib_view.rccl_hip_record_sort_workspace_bytes.argtypes = [c.c_uint32, sz, sz, c.POINTER(sz)]
    lib_view.rccl_hip_record_sort.restype = st
    lib_view.rccl_hip_record_sort.argtypes = [c.c_uint32, sz, vp, vp, vp, vp, sz, vp, sz, vp]
    lib_view.rccl_hip_set_op_workspace_bytes.restype = st
    lib_view.rccl_hip_set_op_workspace_bytes.argtypes = [st, st, sz, sz, sz, c.POINTER(sz)]
    lib_view.rccl_hip_set_op.restype = st
    lib_view.rccl_hip_set_op.argtypes = [st, st, sz, st, vp, vp, sz, vp, vp, sz, vp, vp, sz, vp, vp,
                                         sz, vp]
    lib_view.rccl_hip_group_workspace_bytes.restype = st
    lib_view.rccl_hip_group_workspace_bytes.argtypes = [st, c.c_uint32, st, sz, sz,
                                                        c.POINTER(sz)]
    lib_view.rccl_hip_unique_copy.restype = st
    lib_view.rccl_hip_unique_copy.argtypes = [st, c.c_uint32, sz, vp, vp, vp, vp, sz, vp, vp, sz,
                                              vp]
    lib_view.rccl_hip_reduce_by_key.restype = st
    lib_view.rccl_hip_reduce_by_key.argtypes = [st, c.c_uint32, st, sz, vp, vp, vp, vp, vp, vp,
                                                sz, vp, vp, sz, vp]
    lib_view.rccl_hip_bound_search.restype = st
    lib_view.rccl_hip_bound_search.argtypes = [st, c.c_uint32, st, c.c_int, vp, sz, vp, sz, vp,
                                               vp, sz, vp]
    lib_view.rccl_hip_bound_search_workspace_bytes.restype = st
    lib_view.rccl_hip_bound_search_workspace_bytes.argtypes = [st, c.c_uint32, sz, c.POINTER(sz)]
    lib_view.rccl_hip_set_op_arithmetic.restype = st
    lib_view.rccl_hip_set_op_arithmetic.argtypes = [st, st, st, vp, vp, sz, vp, vp, sz, vp, sz, vp,
                                                    vp, sz, vp]


def load():
    """Load librccl_hip.so (once). Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m rccl_amd.build` "
            "(there is no fallback implementation)")
    try:  # share PyTorch's HIP runtime when both live in one process
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(LIB_PATH)
    _declare(lib)
    _lib = lib
    return lib


def check(status: int) -> None:
    """Raise DeviceAlgorithmError for a failing status."""
    if status != SUCCESS:
        info = ErrorInfo()
        load().rccl_hip_last_error(ctypes.byref(info))
        raise DeviceAlgorithmError(status, info)


def workspace_bytes(fn_name: str, *args) -> int:
    out = ctypes.c_size_t(0)
    check(getattr(load(), fn_name)(*args, ctypes.byref(out)))
    return int(out.value)


def timing_enable(on: bool) -> None:
    check(load().rccl_hip_timing_enable(1 if on else 0))


def timing_read(capacity: int = 1 << 16) -> list:
    """Synchronize and return [(kernel, ms, items)] for the launches recorded
    since the last read (at most `capacity`), clearing the log."""
    lib = load()
    buf = (KernelTiming * capacity)()
    count = ctypes.c_size_t(0)
    check(lib.rccl_hip_timing_read(buf, capacity, ctypes.byref(count)))
    n = min(int(count.value), capacity)
    return [(buf[i].kernel.decode(), float(buf[i].ms), int(buf[i].items)) for i in range(n)]
