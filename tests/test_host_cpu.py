"""CPU tests of the host side: the C ABI library loads and exports every
symbol the header declares, validation rejects bad calls before any launch
(no GPU needed), and the Python mirrors and workload generators behave as
the reference's host code does."""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import radix_shapes

from rccl_amd import _abi, cub, workloads
from rccl_amd.device import KIND_DTYPES, kind_of

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rccl_hip.h")
FAKE = ctypes.c_void_p(4096)  # never dereferenced: every call below fails validation first
# Distinct fake buffers, 4 GiB apart, where a call must pass the overlap checks.
P1, P2, P3, P4 = (ctypes.c_void_p(k << 32) for k in (1, 2, 3, 4))


@pytest.fixture(scope="module")
def lib():
    return _abi.load()


def _declared():
    text = open(HEADER).read()
    return re.findall(r"RCCL_HIP_API\s+[^;]*?\b(rccl_hip_\w+)\s*\(", text)


def test_header_symbols_exported(lib):
    names = _declared()
    assert len(names) >= 15
    out = subprocess.run(["nm", "-D", "--defined-only", _abi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    # Nothing beyond the declared C ABI leaks out of the library.
    extra = sorted(n for n in exported if n.startswith("rccl_hip") and n not in names)
    assert not extra, extra
    assert set(_abi.EXPORTED_SYMBOLS) <= set(names)


def test_scatter_probe_library():
    """bench.py's memory-pattern probe is built beside the tests, exports its
    two entry points, and refuses bad arguments before any launch."""
    path = os.path.join(ROOT, "bench_probes", "libscatter_probe.so")
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert {"scatter_probe_launch", "scatter_probe_tile_items"} <= exported
    probe = ctypes.CDLL(path)
    probe.scatter_probe_tile_items.restype = ctypes.c_size_t
    assert probe.scatter_probe_tile_items() == 512 * 34
    probe.scatter_probe_launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                           ctypes.c_int, ctypes.c_void_p]
    assert probe.scatter_probe_launch(FAKE, FAKE, 1, 5, None) == 1   # no such mode
    assert probe.scatter_probe_launch(FAKE, FAKE, 1, -1, None) == 1
    assert probe.scatter_probe_launch(FAKE, FAKE, 0, 1, None) == 1   # no tiles
    assert probe.scatter_probe_launch(FAKE, FAKE, 1 << 20, 0, None) == 1  # past 2^31 keys


def test_status_strings_and_version(lib):
    assert lib.rccl_hip_abi_version() >= 1
    lib.rccl_hip_status_string.restype = ctypes.c_char_p
    assert lib.rccl_hip_status_string(0) == b"success"
    assert b"workspace" in lib.rccl_hip_status_string(2)
    assert b"bit range" in lib.rccl_hip_status_string(3)


def _last():
    info = _abi.ErrorInfo()
    _abi.load().rccl_hip_last_error(ctypes.byref(info))
    return info


def test_radix_validation_before_launch(lib):
    cur = ctypes.c_int(1)
    # Reversed and out-of-key bit windows (rccl-cub/src/radix.rs:364-392).
    for begin, end in [(5, 4), (0, 33), (40, 48)]:
        rc = lib.rccl_hip_radix_sort_buffer(0, 0, 0, FAKE, FAKE, None, None, 100,
                                            ctypes.byref(cur), begin, end, FAKE, 1 << 20, None)
        assert rc == 3
        info = _last()
        assert (info.begin_bit, info.end_bit, info.key_bits) == (begin, end, 32)
    # A workspace smaller than required reports both sizes.
    need = _abi.workspace_bytes("rccl_hip_radix_sort_workspace_bytes", 0, 0, 1000)
    rc = lib.rccl_hip_radix_sort_buffer(0, 0, 0, P1, P2, None, None, 1000, ctypes.byref(cur),
                                        0, 32, FAKE, need - 1, None)
    assert rc == 2
    info = _last()
    assert (info.expected, info.actual) == (need, need - 1)
    # Unsupported key kinds and value widths.
    out = ctypes.c_size_t()
    assert lib.rccl_hip_radix_sort_workspace_bytes(6, 0, 10, ctypes.byref(out)) == 9  # u8
    assert lib.rccl_hip_radix_sort_workspace_bytes(0, 3, 10, ctypes.byref(out)) == 9


def _ptr(x):
    return ctypes.c_void_p(x)


def test_overlapping_buffers_rejected(lib):
    """Buffers a kernel would read and write in one pass are rejected before
    any launch (the reference's borrows rule them out; through the C ABI a
    caller could pass them). Pointers are never dereferenced: every call fails
    validation, and the accepted layouts fail later on a short workspace."""
    base = 1 << 32
    cur = ctypes.c_int(1)
    n = 1000  # u32 keys: 4,000 bytes
    # Radix double buffer: aliased or partly overlapping halves (keys or values).
    for k1, k2, v1, v2 in [(base, base, None, None), (base, base + 4, None, None),
                           (base, base + 8192, base + 100, base + 20000),
                           (base, base + 8192, base + 16384, base + 16384 + 16)]:
        vb = 0 if v1 is None else 4
        rc = lib.rccl_hip_radix_sort_buffer(0, vb, 0, _ptr(k1), _ptr(k2),
                                            None if v1 is None else _ptr(v1),
                                            None if v2 is None else _ptr(v2), n,
                                            ctypes.byref(cur), 0, 32, FAKE, 1 << 20, None)
        assert rc == 9 and _last().role == b"radix buffers overlap"
    # Disjoint halves pass that check and stop at the workspace.
    assert lib.rccl_hip_radix_sort_buffer(0, 0, 0, _ptr(base), _ptr(base + 4000), None, None, n,
                                          ctypes.byref(cur), 0, 32, FAKE, 1, None) == 2
    # In-place radix sort whose scratch is the keys.
    assert lib.rccl_hip_radix_sort(0, 0, 0, _ptr(base), None, _ptr(base), None, n, FAKE,
                                   1 << 20, None) == 9
    # Merge: an output over an input.
    assert lib.rccl_hip_merge(0, 0, 0, _ptr(base), None, n, _ptr(base + 8192), None, n,
                              _ptr(base + 8192 + 400), None, FAKE, 1 << 20, None) == 9
    assert _last().role == b"merge output overlaps an input"
    # Merge sort: a partly overlapping output is rejected; in place is not.
    assert lib.rccl_hip_merge_sort(0, 0, 0, _ptr(base), None, _ptr(base + 4), None, 100_000,
                                   FAKE, 1 << 30, None) == 9
    assert lib.rccl_hip_merge_sort(0, 0, 0, _ptr(base), None, _ptr(base), None, 100_000,
                                   FAKE, 1, None) == 2
    # Merge sort pairs (copy form): an output over the other stream's input,
    # or the two outputs over each other. u32 keys and values: 400,000 bytes
    # per stream.
    k_in, v_in, k_out, v_out = base, base + (1 << 20), base + (2 << 20), base + (3 << 20)
    for ki, vi, ko, vo in [(k_in, v_in, k_out, k_in + 4000),   # values out over keys in
                           (k_in, v_in, v_in + 400, v_out),    # keys out over values in
                           (k_in, v_in, k_out, k_out + 4)]:    # outputs over each other
        assert lib.rccl_hip_merge_sort(0, 4, 0, _ptr(ki), _ptr(vi), _ptr(ko), _ptr(vo), 100_000,
                                       FAKE, 1 << 30, None) == 9
        assert _last().role == b"merge sort buffers overlap"
    # Disjoint copies, and both streams in place, pass that check.
    for ki, vi, ko, vo in [(k_in, v_in, k_out, v_out), (k_in, v_in, k_in, v_in)]:
        assert lib.rccl_hip_merge_sort(0, 4, 0, _ptr(ki), _ptr(vi), _ptr(ko), _ptr(vo), 100_000,
                                       FAKE, 1, None) == 2
    # Set operations: an output over the second input, even with a huge capacity.
    for cap in (2 * n, (1 << 64) - 1):
        assert lib.rccl_hip_set_op(0, 0, 0, 0, _ptr(base), None, n, _ptr(base + 8192), None, n,
                                   _ptr(base + 8192 + 4 * (n - 1)), None, cap, FAKE, FAKE,
                                   1 << 20, None) == 9
        assert _last().role == b"set output overlaps an input"


def test_overlapping_buffers_rejected_other_calls(lib):
    """The same rule for compaction, bound search and record sort."""
    base = 1 << 32
    cnt = _ptr(base + (1 << 30))
    n = 1000  # u32 keys: 4,000 bytes; u64 values: 8,000 bytes
    # unique_copy: output keys over the input keys, or over the output payloads.
    assert lib.rccl_hip_unique_copy(0, 1, 0, _ptr(base), None, _ptr(base + 2000), None, n, cnt,
                                    FAKE, 1 << 20, None) == 9
    assert _last().role == b"unique output overlaps an input"
    assert lib.rccl_hip_unique_copy(0, 1, 8, _ptr(base), _ptr(base + 8192), _ptr(base + 20000),
                                    _ptr(base + 20000 + 3996), n, cnt, FAKE, 1 << 20, None) == 9
    # reduce_by_key (u64 NaturalBagAdd values): output values over the input values.
    assert lib.rccl_hip_reduce_by_key(0, 1, 1, 0, _ptr(base), None, _ptr(base + 8192),
                                      _ptr(base + 20000), None, _ptr(base + 8192 + 7992), n, cnt,
                                      FAKE, 1 << 20, None) == 9
    assert _last().role == b"reduce-by-key output overlaps"
    # Bound search: indices over the needles.
    assert lib.rccl_hip_bound_search(0, 1, 0, 0, _ptr(base), n, _ptr(base + 8192), n,
                                     _ptr(base + 8192 + 16), FAKE, 1 << 20, None) == 9
    assert _last().role == b"search output overlaps an input"
    # Record sort: rows out partly over rows in; in place is accepted.
    assert lib.rccl_hip_record_sort(4, 0, _ptr(base), None, _ptr(base + 16), None, 100_000,
                                    FAKE, 1 << 30, None) == 9
    assert _last().role == b"record-sort buffers overlap"
    assert lib.rccl_hip_record_sort(4, 8, _ptr(base), _ptr(base + (1 << 28)), _ptr(base),
                                    _ptr(base + (1 << 28)), 100_000, FAKE, 1, None) == 2
    # Record sort with payloads: payloads out over rows in, rows out over
    # payloads in (rows of 16 bytes: 1,600,000 bytes; payloads 800,000).
    r_in, p_in, r_out, p_out = base, base + (4 << 20), base + (8 << 20), base + (12 << 20)
    for ri, pi, ro, po in [(r_in, p_in, r_out, r_in + 1000), (r_in, p_in, p_in + 8, p_out)]:
        assert lib.rccl_hip_record_sort(4, 8, _ptr(ri), _ptr(pi), _ptr(ro), _ptr(po), 100_000,
                                        FAKE, 1 << 30, None) == 9
        assert _last().role == b"record-sort buffers overlap"
    assert lib.rccl_hip_record_sort(4, 8, _ptr(r_in), _ptr(p_in), _ptr(r_out), _ptr(p_out),
                                    100_000, FAKE, 1, None) == 2


def test_merge_and_sort_validation(lib):
    huge = (1 << 64) - 1
    assert lib.rccl_hip_merge(0, 0, 0, FAKE, None, huge, FAKE, None, 2, FAKE, None, FAKE, 1,
                              None) == 5  # SizeOverflow
    need = _abi.workspace_bytes("rccl_hip_merge_workspace_bytes", 0, 0, 50_000, 50_000)
    assert lib.rccl_hip_merge(0, 0, 0, P1, None, 50_000, P2, None, 50_000, P3, None, FAKE,
                              need - 1, None) == 2
    assert lib.rccl_hip_merge(0, 4, 0, FAKE, None, 10, FAKE, None, 10, FAKE, None, FAKE,
                              need, None) == 9  # values missing
    assert lib.rccl_hip_merge(0, 0, 0, None, None, 0, None, None, 0, None, None, None, 0,
                              None) == 0  # empty: nothing to do
    need = _abi.workspace_bytes("rccl_hip_merge_sort_workspace_bytes", 3, 8, 100_000)
    assert lib.rccl_hip_merge_sort(3, 8, 0, P1, P2, P3, P4, 100_000, FAKE, need - 1,
                                   None) == 2
    assert lib.rccl_hip_merge_sort(3, 8, 2, FAKE, FAKE, FAKE, FAKE, 10, FAKE, need, None) == 9


def test_set_validation(lib):
    assert lib.rccl_hip_set_op(9, 0, 0, 0, FAKE, None, 10, FAKE, None, 10, FAKE, None, 20, FAKE,
                               FAKE, 1 << 20, None) == 9  # unknown operation
    assert lib.rccl_hip_set_op(0, 0, 0, 0, FAKE, None, 10, FAKE, None, 10, None, None, 0, None,
                               FAKE, 1 << 20, None) == 9  # count-only needs a count
    need = _abi.workspace_bytes("rccl_hip_set_op_workspace_bytes", 0, 3, 0, 1 << 20, 1 << 20)
    assert lib.rccl_hip_set_op(0, 3, 0, 0, P1, None, 1 << 20, P2, None, 1 << 20, P3, None,
                               1 << 21, FAKE, FAKE, need - 1, None) == 2
    # Union reads the second range's values; intersection does not.
    assert lib.rccl_hip_set_op(0, 0, 4, 0, FAKE, FAKE, 10, FAKE, None, 10, FAKE, FAKE, 20, FAKE,
                               FAKE, 1 << 20, None) == 9


def test_set_arithmetic_validation(lib):
    one = ctypes.c_int64(1)
    p1 = ctypes.byref(one)
    need = _abi.workspace_bytes("rccl_hip_set_op_workspace_bytes", 0, 4, 0, 300, 300)
    # Floating keys have no arithmetic ranges.
    assert lib.rccl_hip_set_op_arithmetic(0, 2, 0, p1, p1, 10, p1, p1, 10, FAKE, 20, FAKE, FAKE,
                                          need, None) == 9
    # Every index must fit the key type: u8 holds 256 items, i8 128.
    assert lib.rccl_hip_set_op_arithmetic(0, 6, 0, p1, p1, 257, p1, p1, 10, FAKE, 300, FAKE,
                                          FAKE, need, None) == 9
    info = _last()
    assert info.role == b"first arithmetic range index" and (info.expected, info.actual) == (
        256, 257)
    assert lib.rccl_hip_set_op_arithmetic(0, 7, 0, p1, p1, 10, p1, p1, 129, FAKE, 300, FAKE,
                                          FAKE, need, None) == 9
    assert _last().role == b"second arithmetic range index"
    # Missing start/step, missing output and count, short workspace.
    assert lib.rccl_hip_set_op_arithmetic(0, 4, 0, None, p1, 10, p1, p1, 10, FAKE, 20, FAKE,
                                          FAKE, need, None) == 9
    assert lib.rccl_hip_set_op_arithmetic(0, 4, 0, p1, p1, 10, p1, p1, 10, None, 0, None, FAKE,
                                          need, None) == 9
    big = _abi.workspace_bytes("rccl_hip_set_op_workspace_bytes", 0, 4, 0, 1 << 20, 1 << 20)
    assert lib.rccl_hip_set_op_arithmetic(0, 4, 0, p1, p1, 1 << 20, p1, p1, 1 << 20, FAKE,
                                          1 << 21, FAKE, FAKE, big - 1, None) == 2
    # Overflowing combined length.
    assert lib.rccl_hip_set_op_arithmetic(0, 4, 0, p1, p1, (1 << 64) - 1, p1, p1, 2, FAKE, 1,
                                          FAKE, FAKE, big, None) == 5


def test_arithmetic_range_host_items():
    r = cub.arithmetic_range(np.uint8(250), np.uint8(3), 4)
    assert r.to_host_vec().tolist() == [250, 253, 0, 3]  # wrapping u8 arithmetic
    r = cub.arithmetic_range(np.int16(100), np.int16(-7), 3)
    assert r.to_host_vec().tolist() == [100, 93, 86]
    r = cub.arithmetic_range(np.int64(-(1 << 62)), np.int64(1 << 61), 5)
    assert r.to_host_vec().tolist() == [-(1 << 62) + k * (1 << 61) for k in range(5)]
    with pytest.raises(TypeError):
        cub.arithmetic_range(np.float32(0), np.float32(1), 3)


def test_group_validation(lib):
    out = ctypes.c_size_t()
    # Keys: scalar kinds at arity 1, u32 rows at arity 2..6.
    assert lib.rccl_hip_group_workspace_bytes(0, 1, 0, 0, 100, ctypes.byref(out)) == 0
    assert lib.rccl_hip_group_workspace_bytes(0, 6, 0, 0, 100, ctypes.byref(out)) == 0
    assert lib.rccl_hip_group_workspace_bytes(0, 7, 0, 0, 100, ctypes.byref(out)) == 9
    assert lib.rccl_hip_group_workspace_bytes(3, 2, 0, 0, 100, ctypes.byref(out)) == 9  # u64 rows
    assert lib.rccl_hip_group_workspace_bytes(0, 1, 4, 0, 100, ctypes.byref(out)) == 9  # operator
    # Payload widths: unique 0/1/2/4/8, reductions 0/4/8.
    assert lib.rccl_hip_group_workspace_bytes(0, 1, 0, 2, 100, ctypes.byref(out)) == 0
    assert lib.rccl_hip_group_workspace_bytes(0, 1, 1, 2, 100, ctypes.byref(out)) == 9
    assert lib.rccl_hip_group_workspace_bytes(0, 1, 0, 16, 100, ctypes.byref(out)) == 9
    need = _abi.workspace_bytes("rccl_hip_group_workspace_bytes", 0, 1, 1, 0, 1 << 20)
    assert 0 < need < (1 << 20)  # look-back state only
    assert lib.rccl_hip_reduce_by_key(0, 1, 1, 0, P1, None, P2, P3, None, P4, 1 << 20,
                                      FAKE, FAKE, need - 1, None) == 2
    assert lib.rccl_hip_reduce_by_key(0, 1, 0, 0, FAKE, None, FAKE, FAKE, None, FAKE, 10, FAKE,
                                      FAKE, need, None) == 9  # UNIQUE is not a reduction
    assert lib.rccl_hip_reduce_by_key(0, 1, 1, 0, FAKE, None, FAKE, FAKE, None, FAKE, 10, None,
                                      FAKE, need, None) == 9  # count required
    assert lib.rccl_hip_unique_copy(0, 1, 8, FAKE, None, FAKE, FAKE, 10, FAKE, FAKE, need,
                                    None) == 9  # payload pointers required


def test_record_sort_validation(lib):
    out = ctypes.c_size_t()
    # Arity 2..6 only (rccl-thrust/src/record_sort.rs:117-126).
    for arity in (0, 1, 7):
        assert lib.rccl_hip_record_sort_workspace_bytes(arity, 0, 10, ctypes.byref(out)) == 4
        info = _last()
        assert b"arities 2 through 6" in info.role and b"use radix sort" in info.role
        assert lib.rccl_hip_record_sort(arity, 0, FAKE, None, FAKE, None, 10, FAKE, 1 << 20,
                                        None) == 4
    # Payloads are u64/f64 (8 bytes) or BooleanProvenance (1 byte).
    for width in (2, 4, 16):
        assert lib.rccl_hip_record_sort_workspace_bytes(3, width, 10, ctypes.byref(out)) == 9
    need = _abi.workspace_bytes("rccl_hip_record_sort_workspace_bytes", 4, 8, 100_000)
    assert need >= 100_000 * (16 + 8)  # scratch rows and payloads
    assert lib.rccl_hip_record_sort(4, 8, P1, P2, P1, P2, 100_000, FAKE, need - 1,
                                    None) == 2
    assert (_last().expected, _last().actual) == (need, need - 1)
    assert lib.rccl_hip_record_sort(4, 8, FAKE, None, FAKE, FAKE, 10, FAKE, need, None) == 9
    assert lib.rccl_hip_record_sort(4, 0, None, None, None, None, 0, None, 0, None) == 0
    for arity in range(2, 7):
        small = _abi.workspace_bytes("rccl_hip_record_sort_workspace_bytes", arity, 0, 1000)
        assert small >= 1000 * 4 * arity


def test_record_sort_contract_errors_before_device_work():
    """The reference's contract errors (rccl-thrust/examples/record_sort.rs:164-201),
    raised before any buffer is touched, so host tensors stand in for device ones."""
    import torch

    from rccl_amd import record_sort as rs
    from rccl_amd.device import DeviceBuffer

    def rows(arity, n):
        return rs.RowBuffer(DeviceBuffer(torch.zeros(max(arity * n, 1), dtype=torch.int32),
                                         np.uint32, arity * n), arity, n)

    def buf(dtype, n):
        return DeviceBuffer(torch.zeros(max(n, 1), dtype=torch.int64), dtype, n)

    ex = None  # never reached: validation fails first
    with pytest.raises(_abi.DeviceAlgorithmError, match="record-sort payload"):
        rs.sort_rows_with_payload_lexicographic(ex, rows(2, 3), buf(np.uint64, 2))
    with pytest.raises(_abi.DeviceAlgorithmError, match="record-sort output"):
        rs.sort_rows_lexicographic_into(ex, rows(2, 3), rows(2, 2))
    with pytest.raises(_abi.DeviceAlgorithmError, match="output payload"):
        rs.sort_rows_with_payload_lexicographic_into(ex, rows(2, 3), buf(np.uint64, 3),
                                                     rows(2, 3), buf(np.uint64, 2))
    with pytest.raises(_abi.DeviceAlgorithmError, match="output rows"):
        rs.sort_rows_with_payload_lexicographic_into(ex, rows(2, 3), buf(np.uint64, 3),
                                                     rows(2, 4), buf(np.uint64, 3))
    with pytest.raises(_abi.DeviceAlgorithmError, match="input payload"):
        rs.sort_rows_with_payload_lexicographic_into(ex, rows(2, 3), buf(np.uint64, 4),
                                                     rows(2, 3), buf(np.uint64, 3))
    with pytest.raises(_abi.DeviceAlgorithmError, match="use radix sort for scalar keys") as e:
        rs.sort_rows_lexicographic(ex, rows(1, 3))
    assert e.value.kind == "UnsupportedTarget"
    with pytest.raises(_abi.DeviceAlgorithmError, match="arities 2 through 6"):
        rs.sort_rows_lexicographic(ex, rows(7, 1))
    # Arity is checked before lengths, as in the reference.
    with pytest.raises(_abi.DeviceAlgorithmError, match="arities 2 through 6"):
        rs.sort_rows_with_payload_lexicographic(ex, rows(7, 3), buf(np.uint64, 2))
    # Only the sealed payload set is accepted.
    with pytest.raises(TypeError):
        rs.sort_rows_with_payload_lexicographic(ex, rows(2, 3), buf(np.uint32, 3))


def test_workspace_sizes_scale(lib):
    small = _abi.workspace_bytes("rccl_hip_radix_sort_workspace_bytes", 0, 0, 1 << 10)
    big = _abi.workspace_bytes("rccl_hip_radix_sort_workspace_bytes", 0, 0, 1 << 28)
    assert 0 < small < big < (1 << 28)  # control state only, well under the keys themselves
    assert _abi.workspace_bytes("rccl_hip_merge_workspace_bytes", 0, 0, 0, 0) == 0
    ms = _abi.workspace_bytes("rccl_hip_merge_sort_workspace_bytes", 0, 4, 1 << 20)
    assert ms >= (1 << 20) * 8  # scratch keys and values


@pytest.mark.parametrize("key,kb", [(0, 4), (1, 4), (3, 8), (4, 8)])
@pytest.mark.parametrize("vb", [0, 4, 16])
def test_merge_sort_radix_lowering_workspace(lib, key, kb, vb):
    """Integer merge sorts from 65,536 items run as a radix sort: the
    workspace covers the scratch keys and values plus the radix control
    state; below the threshold and for float keys it is the merge sort's."""
    def align(x):
        return (x + 255) // 256 * 256
    for n in (65_536, 1 << 23):
        ms = _abi.workspace_bytes("rccl_hip_merge_sort_workspace_bytes", key, vb, n)
        radix = _abi.workspace_bytes("rccl_hip_radix_sort_workspace_bytes", key, vb, n)
        # The lowering keeps the large tiles; a plain radix sort of up to 512
        # small tiles (below 2^22 items for every key and value width) uses
        # small ones, whose control state is larger.
        if n >= 1 << 23:
            assert ms >= align(n * kb) + align(n * vb) + radix
        else:
            assert ms > align(n * kb) + align(n * vb)
        # Below the threshold: the merge sort's own workspace, no radix state.
        assert _abi.workspace_bytes("rccl_hip_merge_sort_workspace_bytes", key, vb, 65_535) < \
            align(65_535 * kb) + align(65_535 * vb) + radix
    # Too small a workspace fails before any launch.
    need = _abi.workspace_bytes("rccl_hip_merge_sort_workspace_bytes", key, vb, 70_000)
    assert lib.rccl_hip_merge_sort(key, vb, 0, P1, P2 if vb else None, P1,
                                   P2 if vb else None, 70_000, FAKE, need - 1, None) == 2


@pytest.mark.parametrize("key,kb", [(0, 4), (3, 8)])
@pytest.mark.parametrize("vb", [0, 1, 2, 4, 8, 16])
def test_radix_small_tile_threshold(key, kb, vb):
    """Plain sorts of at most 512 small tiles (256 threads x half a large
    tile's items) use them; one item more takes the large tiles, whose
    control state is about a quarter as large (an eighth for pairs)."""
    m = radix_shapes.small_tile_max(kb, vb)
    at = _abi.workspace_bytes("rccl_hip_radix_sort_workspace_bytes", key, vb, m)
    below = _abi.workspace_bytes("rccl_hip_radix_sort_workspace_bytes", key, vb, m - 1)
    above = _abi.workspace_bytes("rccl_hip_radix_sort_workspace_bytes", key, vb, m + 1)
    assert at == below
    assert above * 3 < at


def test_python_mirror_host_logic():
    assert cub.order_code(None) == cub.ASCENDING
    assert cub.order_code(cub.descending) == cub.DESCENDING
    with pytest.raises(ValueError):
        cub.order_code(lambda a, b: 0)
    assert cub.ascending(1, 2) == -1 and cub.descending(1, 2) == 1
    with pytest.raises(_abi.DeviceAlgorithmError) as e:
        cub._check_len("output", 7, 6)
    assert e.value.role == "output" and (e.value.expected, e.value.actual) == (7, 6)
    assert cub.set_output_capacity("intersection", 5, 9) == 5
    assert cub.set_output_capacity("difference", 5, 9) == 5
    assert cub.set_output_capacity("union", 5, 9) == 14
    for k, d in KIND_DTYPES.items():
        assert kind_of(d) == k


def test_workloads_deterministic_and_shaped():
    assert int(workloads.splitmix64(np.array([0], np.uint64))[0]) == 0xE220A8397B1DCDAF
    a = workloads.hash_range(123, 1000, 17)
    b = workloads.hash_range(123, 1017)[17:]
    assert np.array_equal(a, b)
    k = workloads.c1_keys(1 << 12)
    assert k.dtype == np.uint32 and np.array_equal(k, workloads.c1_keys(1 << 12))
    ka, pa, kb, pb = workloads.c4_merge_inputs(1 << 12)
    assert (np.diff(ka.astype(np.int64)) >= 0).all() and (np.diff(kb.astype(np.int64)) >= 0).all()
    assert ka.max() < (1 << 24) and (pb >> 31).all() and not (pa >> 31).any()
    x, y = workloads.c5_inputs(1 << 12)
    assert x.size == y.size == 1 << 12 and x.dtype == np.uint64
    assert (np.diff(x) >= 0).all() and (np.diff(y) >= 0).all()
    c3 = workloads.c3_keys(1 << 14)
    counts = workloads.c3_special_counts(1 << 14)
    bits = c3.view(np.uint32)
    assert int((bits == 0x80000000).sum()) >= counts["-0"]
    assert int((bits == 0x7FC00000).sum()) == counts["nan"]


def test_reference_bench_keys():
    """The reference benchmark's xorshift fill (benchmarks/ordering-reference.cu:23-33) in
    Python integers masked to 64 bits: this checks numpy's wrapping left shifts, the logical
    right shift and the truncation to the low 32 bits."""
    def fill(i):
        m = (1 << 64) - 1
        x = i ^ workloads.REFERENCE_BENCH_SEED
        x ^= (x << 13) & m
        x ^= x >> 7
        x ^= (x << 17) & m
        return x & 0xFFFFFFFF
    k = workloads.reference_bench_u32(1 << 16)
    assert k.dtype == np.uint32 and k.size == 1 << 16
    for i in (0, 1, 2, 255, 256, 12345, (1 << 16) - 1):
        assert int(k[i]) == fill(i), i
    # The keys use the whole 32-bit range and barely repeat.
    assert int(k.max()) >= 1 << 31 and np.unique(k).size > (1 << 16) - 16


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


def _same_bits(t, host):
    import torch  # noqa: F401
    a = t.cpu().numpy()
    return np.array_equal(a.view(np.dtype(f"u{a.dtype.itemsize}")),
                          host.view(np.dtype(f"u{host.dtype.itemsize}")))


def test_device_generators_match_host_on_cpu():
    """The benchmark's device-side generators (run here by torch on the CPU)
    produce exactly the host generators' bits."""
    from rccl_amd import workloads_device as wd
    n = 1 << 14
    assert _same_bits(wd.hash_range(99, n, 5, "cpu"), workloads.hash_range(99, n, 5))
    assert _same_bits(wd.metric_u32_keys(n, "cpu"), workloads.metric_u32_keys(n))
    k, v = wd.metric_pairs(n, "cpu")
    hk, hv = workloads.metric_pairs(n)
    assert _same_bits(k, hk) and _same_bits(v, hv)
    for d, h in zip(wd.c4_merge_inputs(n, "cpu"), workloads.c4_merge_inputs(n)):
        assert _same_bits(d, h)
    assert _same_bits(wd.c4_merge_sort_keys(n, "cpu"), workloads.c4_merge_sort_keys(n))
    for d, h in zip(wd.c5_inputs(n, "cpu"), workloads.c5_inputs(n)):
        assert _same_bits(d, h)


def test_bound_search_workspace_and_validation(lib):
    """The bound search's two-level index: one item per 128-byte haystack chunk
    and one per 128-byte line of those, none while the LDS sample already
    brackets every needle in one chunk; a call that builds it fails before
    any launch when the workspace is short."""
    ws = lambda key, arity, n: _abi.workspace_bytes(  # noqa: E731
        "rccl_hip_bound_search_workspace_bytes", key, arity, n)

    def align(x):
        return (x + 255) // 256 * 256

    def expect(n, item):
        chunk = max(1, 128 // item)
        chunks = -(-n // chunk)
        if chunks <= 16384 // item:  # the LDS sample's size
            return 0
        return align(chunks * item) + align(-(-chunks // chunk) * item)
    assert ws(0, 1, 4096 * 32) == 0            # u32: 4,096 samples x 32 per chunk
    assert ws(0, 1, 4096 * 32 + 1) == align(4097 * 4) + align(129 * 4)
    assert ws(0, 1, 1 << 26) == (1 << 21) * 4 + (1 << 16) * 4  # the benchmark haystack
    assert ws(6, 1, 16384 * 128) == 0          # u8: 16,384 samples x 128 per chunk
    for key, item in [(0, 4), (3, 8), (6, 1), (8, 2), (5, 8)]:
        for n in (1000, 1 << 20, (1 << 26) + 3):
            assert ws(key, 1, n) == expect(n, item), (key, n)
    for arity in range(2, 7):
        assert ws(0, arity, 10_000_000) == expect(10_000_000, 4 * arity), arity
    out = ctypes.c_size_t(0)
    assert lib.rccl_hip_bound_search_workspace_bytes(0, 7, 10, ctypes.byref(out)) == 9
    assert lib.rccl_hip_bound_search_workspace_bytes(42, 1, 10, ctypes.byref(out)) == 9
    n, m = 1 << 26, 1 << 20
    need = ws(0, 1, n)
    assert lib.rccl_hip_bound_search(0, 1, 0, 0, P1, n, P2, m, P3, FAKE, need - 1,
                                     None) == 2
    assert lib.rccl_hip_bound_search(0, 1, 0, 0, P1, n, P2, m, P3, None, 0, None) == 2
    assert lib.rccl_hip_bound_search(0, 1, 0, 0, FAKE, n, FAKE, 0, FAKE, None, 0, None) == 0


def test_comparator_classification():
    """Closures lower to the prebuilt ascending / descending kernels by
    probing, whatever their identity; the reference's custom comparators
    (rccl-thrust/examples/sort.rs:36-49,100-112) and a float total order that
    separates the signed zeros are rejected."""
    import struct

    from rccl_amd import cub

    def rust_cmp(a, b):
        return (a > b) - (a < b)

    for dt in (np.uint8, np.int16, np.uint32, np.int64, np.float32, np.float64):
        assert cub.order_code(lambda a, b: rust_cmp(a, b), dt) == cub.ASCENDING
        assert cub.order_code(lambda a, b: rust_cmp(b, a), dt) == cub.DESCENDING
        assert cub.order_code(lambda a, b: -1 if a < b else (1 if a > b else 0), dt) == 0
    assert cub.order_code(cub.descending) == cub.DESCENDING
    assert cub.order_code(None) == cub.ASCENDING
    assert cub.order_code(cub.DESCENDING) == cub.DESCENDING
    custom = [
        lambda l, r: -1 if (l & 1) == 0 and (r & 1) != 0 else
        (1 if (l & 1) != 0 and (r & 1) == 0 else rust_cmp(l, r)),
        lambda l, r: rust_cmp(l & 1, r & 1) or rust_cmp(l, r),
        lambda l, r: rust_cmp(l // 10, r // 10),
        lambda l, r: 0,
        lambda l, r: rust_cmp(abs(l), abs(r)),
    ]
    for f in custom:
        with pytest.raises(cub.ComparatorNotLowered):
            cub.order_code(f, np.int32)

    def total_cmp(a, b):
        ka, kb = (struct.unpack("<i", struct.pack("<f", x))[0] for x in (a, b))
        ka ^= (ka >> 31) & 0x7FFFFFFF
        kb ^= (kb >> 31) & 0x7FFFFFFF
        return rust_cmp(ka, kb)

    with pytest.raises(cub.ComparatorNotLowered):
        cub.order_code(total_cmp, np.float32)
    with pytest.raises(ValueError):
        cub.order_code(7)


@pytest.mark.parametrize("dt", [np.uint8, np.int16, np.uint32, np.int32, np.uint64, np.int64])
def test_comparator_single_bit_closures_rejected(dt):
    """A closure that agrees with the natural order except through one bit (it
    flips, masks or ignores bit k) is rejected for every bit of the key type:
    the probe keys hold 2^k - 1, 2^k and 2^k + 1 for every k."""
    from rccl_amd import cub

    bits = 8 * np.dtype(dt).itemsize
    signed = np.dtype(dt).kind == "i"
    # (On Python's unbounded integers, flipping or clearing the sign bit of a
    # signed key moves every negative key by the same amount: still the
    # natural order, so that bit is not probed for signed types.)
    for k in range(bits - 1 if signed else bits):
        m = 1 << k
        flip = lambda a, b, m=m: cub.ascending(a ^ m, b ^ m)
        ignore = lambda a, b, m=m: cub.ascending(a & ~m, b & ~m)
        for f in (flip, ignore):
            with pytest.raises(cub.ComparatorNotLowered):
                cub.order_code(f, dt)


def test_comparator_single_bit_float_closures_rejected():
    """The same for float keys compared through their bit patterns with one
    bit of the pattern flipped."""
    import struct

    from rccl_amd import cub

    for fmt, ifmt, bits, dt in (("<f", "<I", 32, np.float32), ("<d", "<Q", 64, np.float64)):
        def key(x, m, fmt=fmt, ifmt=ifmt):
            u = struct.unpack(ifmt, struct.pack(fmt, x))[0] ^ m
            return struct.unpack(fmt, struct.pack(ifmt, u))[0]

        for k in range(bits - 1):
            m = 1 << k
            f = lambda a, b, m=m: cub.ascending(key(a, m), key(b, m))
            with pytest.raises(cub.ComparatorNotLowered):
                cub.order_code(f, dt)


def test_static_radix_rejects_oversized_before_any_launch(lib):
    """rccl_hip_radix_sort_static refuses a sort whose control workspace
    exceeds its static array (48 MiB) with WorkspaceTooSmall before touching
    the device; the error names the need and the limit."""
    limit = 48 << 20
    n = 1 << 31
    need = _abi.workspace_bytes("rccl_hip_radix_sort_workspace_bytes", _abi.KEY_KINDS["u32"], 0, n)
    assert need > limit
    st = lib.rccl_hip_radix_sort_static(_abi.KEY_KINDS["u32"], 0, 0, None, None, None, None, n,
                                        None)
    assert st == 2  # WorkspaceTooSmall
    info = _abi.ErrorInfo()
    lib.rccl_hip_last_error(ctypes.byref(info))
    assert (info.expected, info.actual) == (need, limit)
    assert info.role == b"static radix workspace"
    assert lib.rccl_hip_radix_sort_static(_abi.KEY_KINDS["u32"], 3, 0, None, None, None, None, 5,
                                          None) == 9  # InvalidArgument


def test_radix_configure_validates(lib):
    """The diagnostic mode switch accepts the documented modes only."""
    assert lib.rccl_hip_radix_configure(3, 0) == 9  # InvalidArgument
    assert lib.rccl_hip_radix_configure(0, 2) == 9
    assert lib.rccl_hip_radix_configure(-1, 0) == 9
    for ranking in _abi.RANKING.values():
        for order in _abi.TILE_ORDER.values():
            assert lib.rccl_hip_radix_configure(ranking, order) == 0
    assert lib.rccl_hip_radix_configure(0, 0) == 0


def test_sampled_partition_workspaces(lib):
    """From 512 tiles, integer-key merges and set operations hold one u32
    sample count per 2,048 items of the first input beside the tile splits;
    below that, and for float keys, the workspace holds the splits (and the
    set operations' look-back state) alone. Exact sizes, worked out by hand
    from the layout: 256-byte aligned sections."""
    merge = lambda na, nb, key=0: _abi.workspace_bytes(
        "rccl_hip_merge_workspace_bytes", key, 4, na, nb)
    # u32 keys + u32 values: 2,048-item tiles. 2^19 items = 256 tiles: splits
    # only, (256 + 1) * 8 B -> 2,304 B.
    assert merge(1 << 18, 1 << 18) == 2304
    # 2^23 items = 4,096 tiles: splits 4,097 * 8 B -> 33,024 B, plus 2,048
    # sample counts of 4 B (2^22 / 2,048) -> 41,216 B.
    assert merge(1 << 22, 1 << 22) == 41216
    # f32 keys keep the plain search: splits only.
    assert merge(1 << 22, 1 << 22, key=2) == 33024
    setop = lambda na, nb, key: _abi.workspace_bytes(
        "rccl_hip_set_op_workspace_bytes", 0, key, 0, na, nb)
    # u32 keys only: 8,192-item partition tiles, two per look-back tile,
    # groups of 64 look-back tiles; the look-back state is the descriptors,
    # a 16-word gap, the group aggregates, another 16-word gap, the group
    # prefixes and the ticket. 2^21 items = 256 tiles: splits 257 * 16 B ->
    # 4,352 B, then 128 + 16 + 2 + 16 + 2 + 1 words (1,320 B) -> 5,888 B.
    assert setop(1 << 20, 1 << 20, 0) == 5888
    # 2^23 items = 1,024 tiles: splits 1,025 * 16 B -> 16,640 B, then
    # 512 + 16 + 8 + 16 + 8 + 1 words (4,488 B) -> 21,128 B, aligned to
    # 21,248 B, plus 2,048 sample counts -> 29,440 B; f32 keys: 21,248 B.
    assert setop(1 << 22, 1 << 22, 0) == 29440
    assert setop(1 << 22, 1 << 22, 2) == 21248


def test_radix_wide_descriptors_from_2pow30(lib):
    """From 2^30 items the radix look-back descriptors are 64-bit (a digit's
    prefix count no longer fits in 30 bits). u32 keys only: 512 x 34 = 17,408
    items per tile, so 2^30 - 1 and 2^30 items both make 61,681 tiles in 3,856
    groups of 16; the two look-back buffers each hold 61,681 x 256 tile
    descriptors and 3,856 x 256 group prefixes, which grow by 4 bytes each:
    2 x (61,681 + 3,856) x 256 x 4 = 134,219,776 bytes (every section already
    256-byte aligned); nothing else changes."""
    ws = lambda n: _abi.workspace_bytes("rccl_hip_radix_sort_workspace_bytes", 0, 0, n)
    assert ws(1 << 30) - ws((1 << 30) - 1) == 134_219_776
    assert ws((1 << 30) + 1) - ws(1 << 30) == 0  # the same tile count
