"""Python mirror of the reference's rccl-cub ordering surface over the C ABI.

Names, argument meaning and error behaviour follow rccl-cub (paths relative to
the StarGazerM/rccl tree):
  Program.load / Program.on            rccl-cub/src/cuda.rs:741-771
  device_radix_sort_*                  rccl-cub/src/dispatch.rs:2091-2943
  device_merge_{keys,pairs}            rccl-cub/src/dispatch.rs:1572,1915
  device_merge_sort_*                  rccl-cub/src/dispatch.rs:170-322,1116-1400
  typed workspaces                     rccl-cub/src/workspace.rs:108-706
  DoubleBuffer                         rccl-cub/src/double_buffer.rs:6-130
All calls are stream-ordered and asynchronous, as in CUB; every argument is
validated before the first launch and failures raise DeviceAlgorithmError.
Comparator closures are the two prebuilt orders: pass ``ascending`` /
``descending`` (or ``order.ASCENDING`` / ``order.DESCENDING``).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _abi
from ._abi import DeviceAlgorithmError  # noqa: F401  (re-export)
from .device import DeviceBuffer, kind_of

ASCENDING = _abi.ASCENDING
DESCENDING = _abi.DESCENDING


def ascending(a, b):
    """The natural-order comparator `|a, b| a.cmp(b)`."""
    return (a > b) - (a < b)


def descending(a, b):
    """The reversed comparator `|a, b| b.cmp(a)`."""
    return (b > a) - (b < a)


def order_code(order) -> int:
    """Lower a comparator to its prebuilt kernel variant."""
    if order is None or order is ascending or order == ASCENDING:
        return ASCENDING
    if order is descending or order == DESCENDING:
        return DESCENDING
    raise ValueError("only the ascending and descending orders have prebuilt kernels")


class Program:
    """Loaded kernel program for one device (replaces the embedded module)."""

    def __init__(self, device: int):
        self.device = device

    @staticmethod
    def load(device: int = 0) -> "Program":
        _abi.check(_abi.load().rccl_hip_program_load(device))
        return Program(device)

    def on(self, stream: torch.cuda.Stream | None = None) -> "Launch":
        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        if stream.device.index != self.device:
            # rccl-cub/src/cuda.rs:763-765: the program must match the stream's context.
            raise ValueError("ContextMismatch: stream belongs to another device")
        return Launch(self, stream)


class Launch:
    """A stream-bound launch context (rccl-cub/src/cuda.rs:68-105)."""

    def __init__(self, program: Program, stream: torch.cuda.Stream):
        self.program = program
        self._stream = stream

    def stream(self) -> torch.cuda.Stream:
        return self._stream

    @property
    def handle(self) -> int:
        return self._stream.cuda_stream

    def synchronize(self) -> None:
        self._stream.synchronize()


class DoubleBuffer:
    """Two equal-length ranges plus a selector (rccl-cub/src/double_buffer.rs)."""

    def __init__(self, first, second, current_is_first: bool = True):
        self.first = first
        self.second = second
        self._current_is_first = current_is_first

    @staticmethod
    def new(first: DeviceBuffer, second: DeviceBuffer):
        return DoubleBuffer(first, second) if first.len() == second.len() else None

    @staticmethod
    def paired(first, second):
        n = first[0].len()
        if first[1].len() == n and second[0].len() == n and second[1].len() == n:
            return DoubleBuffer(first, second)
        return None

    def current_is_first(self) -> bool:
        return self._current_is_first

    def current(self):
        return self.first if self._current_is_first else self.second

    def swap(self) -> None:
        self._current_is_first = not self._current_is_first

    def len(self) -> int:
        return (self.first[0] if isinstance(self.first, tuple) else self.first).len()


# ---------------------------------------------------------------------------
# Radix sort workspaces (caller-owned, typed, opaque).
# ---------------------------------------------------------------------------
class DeviceRadixSortBufferWorkspace:
    def __init__(self, key_kind: str, value_bytes: int, n: int, launch: Launch):
        self.key_kind = key_kind
        self.value_bytes = value_bytes
        self.n = n
        nbytes = _abi.workspace_bytes("rccl_hip_radix_sort_workspace_bytes",
                                      _abi.KEY_KINDS[key_kind], value_bytes, n)
        self.control = DeviceBuffer.bytes(nbytes, launch.program.device)
        self.control_bytes = nbytes


class DeviceRadixSortKeysWorkspace(DeviceRadixSortBufferWorkspace):
    def __init__(self, key_kind: str, n: int, launch: Launch):
        super().__init__(key_kind, 0, n, launch)
        self.scratch_keys = DeviceBuffer.zeroed(np.dtype(_kind_dtype(key_kind)), n,
                                                launch.program.device)


class DeviceRadixSortPairsWorkspace(DeviceRadixSortBufferWorkspace):
    def __init__(self, key_kind: str, value_dtype, n: int, launch: Launch):
        value_dtype = np.dtype(value_dtype)
        super().__init__(key_kind, value_dtype.itemsize, n, launch)
        self.scratch_keys = DeviceBuffer.zeroed(np.dtype(_kind_dtype(key_kind)), n,
                                                launch.program.device)
        self.scratch_values = DeviceBuffer.zeroed(value_dtype, n, launch.program.device)


def _kind_dtype(kind: str):
    from .device import KIND_DTYPES
    return KIND_DTYPES[kind]


def _radix_kind(dtype) -> str:
    kind = kind_of(dtype)
    if kind not in _abi.RADIX_KINDS:
        raise TypeError(f"{dtype} is not a RadixKey type")
    return kind


def device_radix_sort_workspace(launch: Launch, key_dtype, n: int):
    return DeviceRadixSortKeysWorkspace(_radix_kind(key_dtype), n, launch)


def device_radix_sort_pairs_workspace(launch: Launch, key_dtype, value_dtype, n: int):
    return DeviceRadixSortPairsWorkspace(_radix_kind(key_dtype), value_dtype, n, launch)


def device_radix_sort_keys_buffer_workspace(launch: Launch, key_dtype, n: int):
    return DeviceRadixSortBufferWorkspace(_radix_kind(key_dtype), 0, n, launch)


def device_radix_sort_pairs_buffer_workspace(launch: Launch, key_dtype, value_dtype, n: int):
    return DeviceRadixSortBufferWorkspace(_radix_kind(key_dtype), np.dtype(value_dtype).itemsize,
                                          n, launch)


def _check_len(role: str, expected: int, actual: int) -> None:
    if expected != actual:
        info = _abi.ErrorInfo()
        info.status, info.role, info.expected, info.actual = 1, role.encode(), expected, actual
        raise DeviceAlgorithmError(1, info)


def _radix_inplace(launch, keys, values, ws, order):
    kind = _radix_kind(keys.dtype)
    n = keys.len()
    _check_len("radix scratch keys", n, ws.scratch_keys.len())
    vb, vptr, sptr = 0, None, None
    if values is not None:
        _check_len("radix values", n, values.len())
        _check_len("radix scratch values", n, ws.scratch_values.len())
        vb, vptr, sptr = values.dtype.itemsize, values.ptr, ws.scratch_values.ptr
    _abi.check(_abi.load().rccl_hip_radix_sort(
        _abi.KEY_KINDS[kind], vb, order, keys.ptr, vptr, ws.scratch_keys.ptr, sptr, n,
        ws.control.ptr, ws.control_bytes, launch.handle))


def device_radix_sort_keys(launch, keys, workspace):
    _radix_inplace(launch, keys, None, workspace, ASCENDING)


def device_radix_sort_keys_descending(launch, keys, workspace):
    _radix_inplace(launch, keys, None, workspace, DESCENDING)


def device_radix_sort_pairs(launch, keys, values, workspace):
    _radix_inplace(launch, keys, values, workspace, ASCENDING)


def device_radix_sort_pairs_descending(launch, keys, values, workspace):
    _radix_inplace(launch, keys, values, workspace, DESCENDING)


def _radix_buffer(launch, buffers: DoubleBuffer, bit_range, ws, order, pairs: bool):
    if pairs:
        (k0, v0), (k1, v1) = buffers.first, buffers.second
        vb = v0.dtype.itemsize
        vp0, vp1 = v0.ptr, v1.ptr
    else:
        k0, k1 = buffers.first, buffers.second
        vb, vp0, vp1 = 0, None, None
    kind = _radix_kind(k0.dtype)
    begin, end = bit_range.start, bit_range.stop
    cur = ctypes.c_int(1 if buffers.current_is_first() else 0)
    _abi.check(_abi.load().rccl_hip_radix_sort_buffer(
        _abi.KEY_KINDS[kind], vb, order, k0.ptr, k1.ptr, vp0, vp1, k0.len(), ctypes.byref(cur),
        begin, end, ws.control.ptr, ws.control_bytes, launch.handle))
    buffers._current_is_first = bool(cur.value)


def device_radix_sort_keys_buffer(launch, buffers, bit_range, workspace):
    _radix_buffer(launch, buffers, bit_range, workspace, ASCENDING, False)


def device_radix_sort_keys_buffer_descending(launch, buffers, bit_range, workspace):
    _radix_buffer(launch, buffers, bit_range, workspace, DESCENDING, False)


def device_radix_sort_pairs_buffer(launch, buffers, bit_range, workspace):
    _radix_buffer(launch, buffers, bit_range, workspace, ASCENDING, True)


def device_radix_sort_pairs_buffer_descending(launch, buffers, bit_range, workspace):
    _radix_buffer(launch, buffers, bit_range, workspace, DESCENDING, True)
