"""Python mirror of the reference's rccl-cub ordering surface over the C ABI.

Names, argument meaning and error behaviour follow rccl-cub (paths relative to
the StarGazerM/rccl tree):
  Program.load / Program.on            rccl-cub/src/cuda.rs:741-771
  device_radix_sort_*                  rccl-cub/src/dispatch.rs:2091-2943
  device_merge_{keys,pairs}            rccl-cub/src/dispatch.rs:1572,1915
  device_merge_sort_*                  rccl-cub/src/dispatch.rs:170-322,1116-1400
  device_set_{keys,pairs}              rccl-cub/src/set_operation.rs:265-589 (the
                                       four operations; output=None counts only)
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


class ComparatorNotLowered(ValueError):
    """A comparator closure that is neither the natural order nor its reverse
    on the probe keys. Only those two orders have prebuilt kernels, and there
    is no host fallback, so the call is rejected before any launch."""


def _probe_keys(dtype):
    """Fixed probe keys for classifying a comparator over `dtype`: the type's
    extremes and their neighbours, zero and small values (runs of equal
    decades and both parities), byte boundaries, and for every bit k the
    values 2^k - 1, 2^k and 2^k + 1 (and their negatives for signed types),
    so that a closure that flips or masks one bit disagrees with the natural
    order on some pair; for floats also the infinities, signed zeros,
    denormals, the smallest normals, and every single-bit pattern with
    either sign."""
    dt = np.dtype(dtype)
    bits = 8 * dt.itemsize
    if dt.kind == "f":
        fi = np.finfo(dt)
        tiny, sub = float(fi.tiny), float(fi.smallest_subnormal)
        vals = [-np.inf, -float(fi.max), -1.5, -1.0, -tiny, -sub, -0.0, 0.0, sub, tiny, 0.5,
                1.0, 1.5, 2.0, 10.0, 14.0, 15.0, 16.0, 25.0, 26.0, float(fi.max), np.inf]
        ut = np.dtype(f"u{dt.itemsize}")
        single = np.array([1 << k for k in range(bits - 1)], dtype=ut).view(dt)
        single = single[np.isfinite(single)]
        vals += [float(v) for v in single] + [-float(v) for v in single]
    else:
        ii = np.iinfo(dt)
        small = list(range(0, 22)) + [126, 127, 128, 129, 255, 256]
        vals = [ii.min, ii.min + 1, ii.max - 1, ii.max, ii.max // 2, ii.max // 2 + 1]
        vals += [v for v in small if v <= ii.max]
        for k in range(bits):
            vals += [v for v in ((1 << k) - 1, 1 << k, (1 << k) + 1) if v <= ii.max]
        if ii.min < 0:
            vals += [-v for v in vals if v > 0 and -v >= ii.min]
    # Distinct bit patterns (-0.0 and +0.0 both stay), as Python scalars
    # (float keys widen exactly), which is what a Python closure expects.
    arr = np.array(vals, dtype=dt)
    _, first = np.unique(arr.view(f"u{dt.itemsize}"), return_index=True)
    conv = float if dt.kind == "f" else int
    return [conv(arr[i]) for i in sorted(first)]


def _sign(x) -> int:
    return (x > 0) - (x < 0)


def order_code(order, dtype=None) -> int:
    """Lower a comparator to its prebuilt kernel variant.

    ``ascending`` / ``descending`` (or the ABI codes) map directly. Any other
    closure ``f(a, b) -> negative | 0 | positive`` (Rust's Ordering as a
    sign) is classified by evaluating it on every pair of the probe keys of
    ``dtype``: if it agrees with the natural order everywhere it lowers to
    ASCENDING, if with the reversed order DESCENDING; otherwise
    ComparatorNotLowered is raised. For floats the natural order is IEEE
    comparison, so -0.0 and +0.0 are equivalent: a closure that orders them
    (Rust's total_cmp) is rejected rather than silently changed."""
    if order is None or order is ascending:
        return ASCENDING
    if order is descending:
        return DESCENDING
    if isinstance(order, (int, np.integer)) and not isinstance(order, bool):
        if int(order) in (ASCENDING, DESCENDING):
            return int(order)
        raise ValueError(f"unknown order code {order}")
    if not callable(order):
        raise TypeError("an order is a comparator closure or an order code")
    probes = _probe_keys(np.uint32 if dtype is None else dtype)
    asc = desc = True
    for a in probes:
        for b in probes:
            got = _sign(order(a, b))
            nat = _sign(ascending(a, b))
            asc = asc and got == nat
            desc = desc and got == -nat
            if not (asc or desc):
                raise ComparatorNotLowered(
                    "the comparator is neither the natural order nor its reverse on the probe "
                    f"keys (it returned {got} for ({a!r}, {b!r})); only those orders have "
                    "prebuilt kernels")
    return ASCENDING if asc else DESCENDING


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


# ---------------------------------------------------------------------------
# DeviceMerge (rccl-cub/src/merge.rs:194-368, dispatch.rs:1572,1915).
# ---------------------------------------------------------------------------
def _ordering_kind(dtype) -> str:
    kind = kind_of(dtype)
    if kind not in _abi.KEY_KINDS:
        raise TypeError(f"{dtype} has no prebuilt ordering kernels")
    return kind


def _value_bytes(value_dtype) -> int:
    return 0 if value_dtype is None else np.dtype(value_dtype).itemsize


class DeviceMergeWorkspace:
    """Caller-owned partition storage for one merge shape."""

    def __init__(self, launch: Launch, key_dtype, na: int, nb: int, value_dtype=None):
        self.key_kind = _ordering_kind(key_dtype)
        self.value_bytes = _value_bytes(value_dtype)
        self.na, self.nb = na, nb
        self.control_bytes = _abi.workspace_bytes(
            "rccl_hip_merge_workspace_bytes", _abi.KEY_KINDS[self.key_kind], self.value_bytes,
            na, nb)
        self.control = DeviceBuffer.bytes(self.control_bytes, launch.program.device)


def device_merge_workspace(launch, key_dtype, na, nb):
    return DeviceMergeWorkspace(launch, key_dtype, na, nb)


def device_merge_pairs_workspace(launch, key_dtype, value_dtype, na, nb):
    return DeviceMergeWorkspace(launch, key_dtype, na, nb, value_dtype)


def _ws_ptr(ws):
    return (ws.control.ptr if ws.control_bytes else None), ws.control_bytes


def device_merge_keys(launch, first, second, workspace, output, order=ascending):
    """Stable merge of two sorted ranges; equal keys take `first` first."""
    total = first.len() + second.len()
    _check_len("output", total, output.len())
    kind = _ordering_kind(first.dtype)
    wptr, wbytes = _ws_ptr(workspace)
    _abi.check(_abi.load().rccl_hip_merge(
        _abi.KEY_KINDS[kind], 0, order_code(order, first.dtype), first.ptr, None, first.len(),
        second.ptr, None, second.len(), output.ptr, None, wptr, wbytes, launch.handle))


def device_merge_pairs(launch, first_keys, first_values, second_keys, second_values, workspace,
                       output_keys, output_values, order=ascending):
    _check_len("first values", first_keys.len(), first_values.len())
    _check_len("second values", second_keys.len(), second_values.len())
    total = first_keys.len() + second_keys.len()
    _check_len("output keys", total, output_keys.len())
    _check_len("output values", total, output_values.len())
    kind = _ordering_kind(first_keys.dtype)
    wptr, wbytes = _ws_ptr(workspace)
    _abi.check(_abi.load().rccl_hip_merge(
        _abi.KEY_KINDS[kind], first_values.dtype.itemsize, order_code(order, first_keys.dtype),
        first_keys.ptr,
        first_values.ptr, first_keys.len(), second_keys.ptr, second_values.ptr,
        second_keys.len(), output_keys.ptr, output_values.ptr, wptr, wbytes, launch.handle))


# ---------------------------------------------------------------------------
# DeviceMergeSort (rccl-cub/src/merge_sort.rs:140-690, dispatch.rs:170-322,1116-1400).
# ---------------------------------------------------------------------------
class DeviceMergeSortWorkspace:
    """Caller-owned scratch keys/values and partitions for one sort length."""

    def __init__(self, launch: Launch, key_dtype, n: int, value_dtype=None):
        self.key_kind = _ordering_kind(key_dtype)
        self.value_bytes = _value_bytes(value_dtype)
        self.n = n
        self.control_bytes = _abi.workspace_bytes(
            "rccl_hip_merge_sort_workspace_bytes", _abi.KEY_KINDS[self.key_kind],
            self.value_bytes, n)
        self.control = DeviceBuffer.bytes(self.control_bytes, launch.program.device)


def device_merge_sort_workspace(launch, key_dtype, n):
    return DeviceMergeSortWorkspace(launch, key_dtype, n)


def device_merge_sort_pairs_workspace(launch, key_dtype, value_dtype, n):
    return DeviceMergeSortWorkspace(launch, key_dtype, n, value_dtype)


def _merge_sort(launch, in_keys, in_values, out_keys, out_values, ws, order):
    n = in_keys.len()
    _check_len("merge-sort workspace", ws.n, n)
    kind = _ordering_kind(in_keys.dtype)
    vb = 0 if in_values is None else in_values.dtype.itemsize
    wptr, wbytes = _ws_ptr(ws)
    _abi.check(_abi.load().rccl_hip_merge_sort(
        _abi.KEY_KINDS[kind], vb, order_code(order, in_keys.dtype), in_keys.ptr,
        None if in_values is None else in_values.ptr, out_keys.ptr,
        None if out_values is None else out_values.ptr, n, wptr, wbytes, launch.handle))


def device_merge_sort_keys(launch, keys, workspace, order=ascending):
    """Stable in-place merge sort of `keys`."""
    _merge_sort(launch, keys, None, keys, None, workspace, order)


def device_merge_sort_keys_copy(launch, input, workspace, output, order=ascending):
    _check_len("output keys", input.len(), output.len())
    _merge_sort(launch, input, None, output, None, workspace, order)


def device_merge_sort_pairs(launch, keys, values, workspace, order=ascending):
    _check_len("values", keys.len(), values.len())
    _merge_sort(launch, keys, values, keys, values, workspace, order)


def device_merge_sort_pairs_copy(launch, input_keys, input_values, workspace, output_keys,
                                 output_values, order=ascending):
    n = input_keys.len()
    _check_len("input values", n, input_values.len())
    _check_len("output keys", n, output_keys.len())
    _check_len("output values", n, output_values.len())
    _merge_sort(launch, input_keys, input_values, output_keys, output_values, workspace, order)


# ---------------------------------------------------------------------------
# Set operations (rccl-cub/src/set_operation.rs:265-589, dispatch.rs:344-1000).
# ---------------------------------------------------------------------------
SET_OPERATIONS = _abi.SET_OPS


def set_output_capacity(operation, na: int, nb: int) -> int:
    """Largest possible output of a set operation over na + nb keys."""
    op = SET_OPERATIONS[operation] if isinstance(operation, str) else operation
    return {0: na + nb, 1: min(na, nb), 2: na, 3: na + nb}[op]


class DeviceSetOperationWorkspace:
    """Caller-owned tile state, partitions and the device output count."""

    def __init__(self, launch: Launch, operation: str, key_dtype, na: int, nb: int,
                 value_dtype=None):
        self.operation = SET_OPERATIONS[operation]
        self.key_kind = _ordering_kind(key_dtype)
        self.value_bytes = _value_bytes(value_dtype)
        self.control_bytes = _abi.workspace_bytes(
            "rccl_hip_set_op_workspace_bytes", self.operation, _abi.KEY_KINDS[self.key_kind],
            self.value_bytes, na, nb)
        self.control = DeviceBuffer.bytes(self.control_bytes, launch.program.device)
        self.output_count = DeviceBuffer.zeroed(np.dtype(np.uint64), 1, launch.program.device)

    def count(self) -> int:
        """Read the last operation's output length (synchronizes)."""
        return int(self.output_count.to_host_vec()[0])


def device_set_workspace(launch, operation, key_dtype, na, nb):
    return DeviceSetOperationWorkspace(launch, operation, key_dtype, na, nb)


def device_set_pairs_workspace(launch, operation, key_dtype, value_dtype, na, nb):
    return DeviceSetOperationWorkspace(launch, operation, key_dtype, na, nb, value_dtype)


def _set_op(launch, op, first_keys, first_values, second_keys, second_values, ws, output_keys,
            output_values, order):
    kind = _ordering_kind(first_keys.dtype)
    vb = 0
    if output_keys is not None and first_values is not None:
        _check_len("first set values", first_keys.len(), first_values.len())
        if op in (0, 3):
            _check_len("second set values", second_keys.len(), second_values.len())
        _check_len("set output values", output_keys.len(), output_values.len())
        vb = first_values.dtype.itemsize
    _abi.check(_abi.load().rccl_hip_set_op(
        op, _abi.KEY_KINDS[kind], vb, order_code(order, first_keys.dtype), first_keys.ptr,
        None if first_values is None else first_values.ptr, first_keys.len(), second_keys.ptr,
        None if second_values is None else second_values.ptr, second_keys.len(),
        None if output_keys is None else output_keys.ptr,
        None if output_values is None or vb == 0 else output_values.ptr,
        0 if output_keys is None else output_keys.len(), ws.output_count.ptr, ws.control.ptr, ws.control_bytes, launch.handle))


def device_set_keys(launch, operation, first, second, workspace, output=None, order=ascending):
    """Enqueue a keys-only set operation; `output=None` only counts. The
    length lands in `workspace.output_count` (device)."""
    _set_op(launch, SET_OPERATIONS[operation], first, None, second, None, workspace, output,
            None, order)


class ArithmeticRange:
    """Finite arithmetic input range: item i is start + step * i in the key
    type's wrapping arithmetic; never materialised (rccl-cub/src/range.rs:43-78)."""

    def __init__(self, start, step, length: int, dtype=None):
        self.dtype = np.dtype(dtype if dtype is not None else np.asarray(start).dtype)
        if self.dtype.kind not in "iu":
            raise TypeError(f"arithmetic ranges have integer items, not {self.dtype}")
        self.start = np.asarray(start).astype(self.dtype)
        self.step = np.asarray(step).astype(self.dtype)
        self._len = int(length)

    def len(self) -> int:
        return self._len

    def __len__(self) -> int:
        return self._len

    def to_host_vec(self) -> np.ndarray:
        """The items, computed on the host in the same wrapping arithmetic."""
        wide = np.uint64
        i = np.arange(self._len, dtype=wide)
        v = self.start.astype(self.dtype).view(f"u{self.dtype.itemsize}").astype(wide) + \
            self.step.astype(self.dtype).view(f"u{self.dtype.itemsize}").astype(wide) * i
        return v.astype(f"u{self.dtype.itemsize}").view(self.dtype)


def arithmetic_range(start, step, length: int, dtype=None) -> ArithmeticRange:
    return ArithmeticRange(start, step, length, dtype)


def device_set_arithmetic(launch, operation, first: ArithmeticRange, second: ArithmeticRange,
                          workspace, output=None, order=ascending):
    """Enqueue a set operation over two arithmetic ranges (keys only);
    `output=None` only counts (rccl-cub/src/dispatch.rs:552-740)."""
    if first.dtype != second.dtype:
        raise TypeError("both arithmetic ranges must have the same item type")
    kind = _ordering_kind(first.dtype)
    a0 = np.ascontiguousarray(np.array([first.start, first.step], dtype=first.dtype))
    b0 = np.ascontiguousarray(np.array([second.start, second.step], dtype=second.dtype))
    w = first.dtype.itemsize
    _abi.check(_abi.load().rccl_hip_set_op_arithmetic(
        SET_OPERATIONS[operation], _abi.KEY_KINDS[kind], order_code(order, first.dtype),
        a0.ctypes.data, a0.ctypes.data + w, first.len(), b0.ctypes.data, b0.ctypes.data + w,
        second.len(), None if output is None else output.ptr,
        0 if output is None else output.len(), workspace.output_count.ptr, workspace.control.ptr,
        workspace.control_bytes, launch.handle))


def device_set_pairs(launch, operation, first_keys, first_values, second_keys, second_values,
                     workspace, output_keys, output_values, order=ascending):
    _set_op(launch, SET_OPERATIONS[operation], first_keys, first_values, second_keys,
            second_values, workspace, output_keys, output_values, order)
