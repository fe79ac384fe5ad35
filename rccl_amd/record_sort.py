"""Python mirror of rccl-thrust's record sort (rccl-thrust/src/record_sort.rs).

Stable ascending lexicographic sort of padding-free ``[u32; N]`` relation rows
(SRDatalog/HISA ``Row<N>``), optionally carrying one provenance payload per
row. Names, argument meaning and error behaviour follow the reference:

  sort_rows_lexicographic                     record_sort.rs:144-185
  sort_rows_lexicographic_into                record_sort.rs:188-227
  sort_rows_with_payload_lexicographic        record_sort.rs:229-279
  sort_rows_with_payload_lexicographic_into   record_sort.rs:281-350

Arity must be 2 through 6 (record_sort.rs:117-126); payloads are the sealed
``RecordPayload`` set u64, f64 and BooleanProvenance (one byte, 0 or 1)
(record_sort.rs:17-31). Every call validates (arity first, then lengths in the
reference's order and with its role strings), allocates its workspace on the
device, runs on the execution's stream and waits for completion, as the
reference's synchronous wrappers do (``...?.wait()``).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _abi
from .cub import _check_len
from .device import DeviceBuffer

MIN_ARITY, MAX_ARITY = 2, 6

# The sealed RecordPayload set (record_sort.rs:17-31). BooleanProvenance is a
# one-byte 0/1 value (rccl-cub/src/grouped_reduction.rs:45-57).
PAYLOAD_DTYPES = (np.dtype(np.uint64), np.dtype(np.float64), np.dtype(np.bool_),
                  np.dtype(np.uint8))


class RowBuffer:
    """Device buffer of ``len`` rows of ``arity`` u32 columns, row-major and
    padding-free (``DeviceBuffer<RelationRow<N>>``)."""

    def __init__(self, words: DeviceBuffer, arity: int, length: int):
        if arity < 1:
            raise ValueError("a row has at least one column")
        self.words = words
        self.arity = int(arity)
        self._len = int(length)

    @staticmethod
    def from_host(rows, device: int = 0) -> "RowBuffer":
        a = np.ascontiguousarray(np.asarray(rows, dtype=np.uint32))
        if a.ndim != 2:
            raise ValueError("rows must be a (len, arity) array")
        return RowBuffer(DeviceBuffer.from_host(a.reshape(-1), device=device), a.shape[1],
                         a.shape[0])

    @staticmethod
    def zeroed(arity: int, length: int, device: int = 0) -> "RowBuffer":
        return RowBuffer(DeviceBuffer.zeroed(np.uint32, arity * length, device), arity, length)

    def len(self) -> int:
        return self._len

    def __len__(self) -> int:
        return self._len

    @property
    def ptr(self) -> int:
        return self.words.ptr

    def to_host_vec(self) -> np.ndarray:
        return self.words.to_host_vec().reshape(self._len, self.arity)


def _payload_bytes(payloads) -> int:
    if payloads is None:
        return 0
    if payloads.dtype not in PAYLOAD_DTYPES:
        raise TypeError(f"record payloads are u64, f64 or BooleanProvenance, not {payloads.dtype}")
    return payloads.dtype.itemsize


def _workspace(execution, arity: int, payload_bytes: int, n: int) -> DeviceBuffer | None:
    nbytes = _abi.workspace_bytes("rccl_hip_record_sort_workspace_bytes", arity, payload_bytes, n)
    if nbytes == 0:
        return None
    return DeviceBuffer.bytes(nbytes, execution.launch().program.device)


def _validate_arity(arity: int, payload_bytes: int) -> None:
    # The library validates the arity (and payload width) without allocating.
    out = ctypes.c_size_t(0)
    _abi.check(_abi.load().rccl_hip_record_sort_workspace_bytes(arity, payload_bytes, 0,
                                                                ctypes.byref(out)))


def _run(execution, in_rows: RowBuffer, in_payloads, out_rows: RowBuffer, out_payloads) -> None:
    pb = _payload_bytes(in_payloads)
    n = in_rows.len()
    ws = _workspace(execution, in_rows.arity, pb, n)
    launch = execution.launch()
    _abi.check(_abi.load().rccl_hip_record_sort(
        in_rows.arity, pb, in_rows.ptr, None if in_payloads is None else in_payloads.ptr,
        out_rows.ptr, None if out_payloads is None else out_payloads.ptr, n,
        None if ws is None else ws.ptr, 0 if ws is None else ws.len(), launch.handle))
    execution.synchronize()


def sort_rows_lexicographic(execution, rows: RowBuffer) -> None:
    """Stably sort ``rows`` in place in ascending lexicographic order."""
    _validate_arity(rows.arity, 0)
    _run(execution, rows, None, rows, None)


def sort_rows_lexicographic_into(execution, input: RowBuffer, output: RowBuffer) -> None:
    """Stable lexicographic sort of ``input`` written to ``output``."""
    _validate_arity(input.arity, 0)
    if output.arity != input.arity:
        raise TypeError("input and output rows have different arities")
    _check_len("record-sort output", input.len(), output.len())
    _run(execution, input, None, output, None)


def sort_rows_with_payload_lexicographic(execution, rows: RowBuffer,
                                         payloads: DeviceBuffer) -> None:
    """Stable in-place sort of ``rows``; ``payloads[i]`` moves with row i."""
    _validate_arity(rows.arity, _payload_bytes(payloads))
    _check_len("record-sort payload", rows.len(), payloads.len())
    _run(execution, rows, payloads, rows, payloads)


def sort_rows_with_payload_lexicographic_into(execution, input_rows: RowBuffer,
                                              input_payloads: DeviceBuffer,
                                              output_rows: RowBuffer,
                                              output_payloads: DeviceBuffer) -> None:
    """Stable sort of rows and payloads into separate output buffers."""
    pb = _payload_bytes(input_payloads)
    _validate_arity(input_rows.arity, pb)
    if output_rows.arity != input_rows.arity:
        raise TypeError("input and output rows have different arities")
    if output_payloads.dtype != input_payloads.dtype:
        raise TypeError("input and output payloads have different types")
    n = input_rows.len()
    _check_len("record-sort input payload", n, input_payloads.len())
    _check_len("record-sort output rows", n, output_rows.len())
    _check_len("record-sort output payload", n, output_payloads.len())
    _run(execution, input_rows, input_payloads, output_rows, output_payloads)
