"""GPU parity tests for the record sort (stable lexicographic [u32; N] rows).

Cases follow the reference's example (rccl-thrust/examples/record_sort.rs):
the payload-stability lengths (:25-55), the arities 2/4/5/6 at 10,003 rows
(:57-76), out-of-place rows with f64 payloads and keys-only arity 6 (:78-122)
and the duplicate-row payload cases (:124-162, also golden vectors). Every
output is compared bit-for-bit with the CPU oracle (oracle_record_sort) on the
same input. The reference's injected comparator trap (:203-229) is not
reproduced: no test here makes the GPU trap on purpose.
"""
import json
import os

import numpy as np
import pytest

import oracle
from rccl_amd import record_sort as rs
from rccl_amd import thrust, workloads
from rccl_amd.device import DeviceBuffer

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("radix_ranking")]

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.json")


@pytest.fixture(scope="module")
def ex():
    return thrust.Program.load(0).par()


def _reference_rows(arity, n):
    """The reference example's row generator (record_sort.rs:11-23)."""
    return workloads.record_rows(arity, n)


def _random_rows(arity, n, seed, distinct=None):
    raw = workloads.hash_range(seed, n * arity).reshape(n, arity)
    if distinct is not None:
        return (raw % np.uint64(distinct)).astype(np.uint32)
    return (raw >> np.uint64(32)).astype(np.uint32)


def _check(ex, rows, payloads=None, into=False):
    exp_rows, exp_payloads = oracle.record_sort(rows, payloads)
    d_rows = rs.RowBuffer.from_host(rows)
    d_pay = None if payloads is None else DeviceBuffer.from_host(payloads)
    if into:
        out_rows = rs.RowBuffer.from_host(np.full_like(rows, 0xFFFFFFFF))
        if d_pay is None:
            rs.sort_rows_lexicographic_into(ex, d_rows, out_rows)
        else:
            out_pay = DeviceBuffer.from_host(np.zeros_like(payloads))
            rs.sort_rows_with_payload_lexicographic_into(ex, d_rows, d_pay, out_rows, out_pay)
            np.testing.assert_array_equal(out_pay.to_host_vec().view(np.uint8),
                                          exp_payloads.view(np.uint8))
        np.testing.assert_array_equal(out_rows.to_host_vec(), exp_rows)
        # Inputs are left untouched.
        np.testing.assert_array_equal(d_rows.to_host_vec(), rows)
        return
    if d_pay is None:
        rs.sort_rows_lexicographic(ex, d_rows)
    else:
        rs.sort_rows_with_payload_lexicographic(ex, d_rows, d_pay)
        np.testing.assert_array_equal(d_pay.to_host_vec().view(np.uint8),
                                      exp_payloads.view(np.uint8))
    np.testing.assert_array_equal(d_rows.to_host_vec(), exp_rows)


@pytest.mark.parametrize("n", [0, 1, 31, 32, 33, 255, 256, 257, 513, 65_537])
def test_stable_payload_boundaries(ex, n):
    """record_sort.rs:25-55: arity 3, payload = input index."""
    rows = _reference_rows(3, n)
    payloads = np.arange(n, dtype=np.uint64)
    _check(ex, rows, payloads)


@pytest.mark.parametrize("arity", [2, 3, 4, 5, 6])
def test_supported_arities(ex, arity):
    """record_sort.rs:57-76 (10,003 rows, keys only)."""
    _check(ex, _reference_rows(arity, 10_003))


def test_out_of_place_f64_payload_and_keys_only(ex):
    """record_sort.rs:78-122."""
    rows = _reference_rows(5, 513)
    payloads = np.arange(513, dtype=np.float64) / 513.0
    _check(ex, rows, payloads, into=True)
    _check(ex, _reference_rows(6, 257), into=True)


def test_golden_vectors(ex):
    cases = [c for c in json.load(open(GOLDEN))["cases"] if c["op"] == "record_sort"]
    assert len(cases) >= 5
    for c in cases:
        rows = np.array(c["rows"], dtype=np.uint32)
        payloads = None
        if "payloads" in c:
            payloads = np.array(c["payloads"], dtype={"u64": np.uint64, "u8": np.bool_}
                                [c["payload_dtype"]])
        d_rows = rs.RowBuffer.from_host(rows)
        if payloads is None:
            rs.sort_rows_lexicographic(ex, d_rows)
        else:
            d_pay = DeviceBuffer.from_host(payloads)
            rs.sort_rows_with_payload_lexicographic(ex, d_rows, d_pay)
            assert d_pay.to_host_vec().astype(np.uint64).tolist() == c["expected_payloads"], c["id"]
        assert d_rows.to_host_vec().tolist() == c["expected_rows"], c["id"]


@pytest.mark.parametrize("arity", [2, 3, 4, 5, 6])
@pytest.mark.parametrize("payload", [None, np.uint64, np.float64, np.bool_])
def test_random_rows_with_ties(ex, arity, payload):
    """Seeded rows over a small alphabet (many equal rows: stability decides
    the payload order) across several merge passes."""
    n = 300_007
    rows = _random_rows(arity, n, 17 + arity, distinct=3)
    pay = None
    if payload is not None:
        raw = workloads.hash_range(99 + arity, n)
        pay = {np.uint64: raw, np.float64: (raw >> np.uint64(11)).astype(np.float64),
               np.bool_: (raw & np.uint64(1)).astype(np.bool_)}[payload]
    _check(ex, rows, pay)
    _check(ex, rows, pay, into=True)


def test_full_range_columns_large(ex):
    """Full-range u32 columns (unsigned order: values above 2^31 sort last),
    2^20 + 13 rows of arity 4 with u64 payloads, the bench workload shape."""
    n = (1 << 20) + 13
    rows = _random_rows(4, n, 4242)
    rows[::7, 0] = rows[::7, 0] & np.uint32(0xF)  # repeated leading columns
    pay = workloads.hash_range(4243, n)
    _check(ex, rows, pay)


def test_sorted_and_reversed_inputs(ex):
    rows = np.sort(_random_rows(3, 100_003, 5, distinct=1000).view("u4,u4,u4"), axis=0)
    rows = rows.view(np.uint32).reshape(-1, 3)
    _check(ex, rows, np.arange(len(rows), dtype=np.uint64))
    _check(ex, rows[::-1].copy(), np.arange(len(rows), dtype=np.uint64))


# ---------------------------------------------------------------------------
# The LSD radix path (65,536 rows and more): pass skipping, the in-place pass
# parity and the buffer roles.
# ---------------------------------------------------------------------------
RADIX_MIN_ROWS = 65_536


def _one_varying_byte(arity, n, seed):
    """Rows whose only non-constant byte is the last column's low byte: one
    active pass, so an in-place sort must activate a trivial one."""
    rows = np.full((n, arity), 0x01020304, dtype=np.uint32)
    rows[:, -1] = (rows[:, -1] & np.uint32(0xFFFFFF00)) | (
        workloads.hash_range(seed, n) & np.uint64(0xFF)).astype(np.uint32)
    return rows


@pytest.mark.parametrize("arity", [2, 3, 4, 5, 6])
def test_radix_single_active_pass(ex, arity):
    n = RADIX_MIN_ROWS + 3
    rows = _one_varying_byte(arity, n, 31 + arity)
    pay = np.arange(n, dtype=np.uint64)
    _check(ex, rows, pay)
    _check(ex, rows, pay, into=True)
    _check(ex, rows)
    _check(ex, rows, into=True)


@pytest.mark.parametrize("arity", [2, 6])
def test_radix_all_rows_equal(ex, arity):
    """No active pass: in place is a no-op, out of place a stable copy."""
    n = RADIX_MIN_ROWS * 2 + 1
    rows = np.full((n, arity), 0xDEADBEEF, dtype=np.uint32)
    pay = workloads.hash_range(77, n)
    _check(ex, rows, pay)
    _check(ex, rows, pay, into=True)


@pytest.mark.parametrize("arity", [2, 3, 4, 5, 6])
@pytest.mark.parametrize("n", [RADIX_MIN_ROWS - 1, RADIX_MIN_ROWS, RADIX_MIN_ROWS + 1])
def test_threshold_sizes(ex, arity, n):
    rows = _random_rows(arity, n, 500 + arity, distinct=7)
    _check(ex, rows, np.arange(n, dtype=np.uint64))


@pytest.mark.parametrize("arity", [2, 4, 6])
def test_radix_every_byte_active(ex, arity):
    """Full-range columns with ties: all 4 * arity passes run."""
    n = 400_009
    rows = _random_rows(arity, n, 900 + arity)
    rows[1::3] = rows[::3][: len(rows[1::3])]  # repeated rows: stability matters
    _check(ex, rows, workloads.hash_range(901 + arity, n))
    _check(ex, rows, workloads.hash_range(901 + arity, n), into=True)


def test_radix_rows_out_of_place_payloads_in_place(ex):
    """Only the payloads alias: the pass plan must still treat the sort as in
    place (rows come back in the output buffer, payloads in their own)."""
    from rccl_amd import _abi

    n, arity = 200_003, 3
    rows = _one_varying_byte(arity, n, 5)
    pay = np.arange(n, dtype=np.uint64)
    exp_rows, exp_pay = oracle.record_sort(rows, pay)
    d_in = rs.RowBuffer.from_host(rows)
    d_out = rs.RowBuffer.zeroed(arity, n)
    d_pay = DeviceBuffer.from_host(pay)
    ws_bytes = _abi.workspace_bytes("rccl_hip_record_sort_workspace_bytes", arity, 8, n)
    ws = DeviceBuffer.bytes(ws_bytes)
    launch = ex.launch()
    _abi.check(_abi.load().rccl_hip_record_sort(arity, 8, d_in.ptr, d_pay.ptr, d_out.ptr,
                                                d_pay.ptr, n, ws.ptr, ws_bytes, launch.handle))
    ex.synchronize()
    np.testing.assert_array_equal(d_out.to_host_vec(), exp_rows)
    np.testing.assert_array_equal(d_pay.to_host_vec(), exp_pay)
    np.testing.assert_array_equal(d_in.to_host_vec(), rows)


@pytest.mark.parametrize("arity", [2, 5])
@pytest.mark.parametrize("alias", ["payloads", "rows"])
def test_radix_all_rows_equal_mixed_aliasing(ex, arity, alias):
    """Every row equal (no pass moves anything) with only one stream in
    place: the other stream's output must still be written, and the aliased
    one left intact."""
    from rccl_amd import _abi

    n = RADIX_MIN_ROWS * 2 + 5
    rows = np.full((n, arity), 0x01020304, dtype=np.uint32)
    pay = workloads.hash_range(91 + arity, n)
    d_in = rs.RowBuffer.from_host(rows)
    d_pay_in = DeviceBuffer.from_host(pay)
    if alias == "payloads":
        d_out, d_pay_out = rs.RowBuffer.zeroed(arity, n), d_pay_in
    else:
        d_out, d_pay_out = d_in, DeviceBuffer.from_host(np.zeros(n, np.uint64))
    ws_bytes = _abi.workspace_bytes("rccl_hip_record_sort_workspace_bytes", arity, 8, n)
    ws = DeviceBuffer.bytes(ws_bytes)
    launch = ex.launch()
    _abi.check(_abi.load().rccl_hip_record_sort(arity, 8, d_in.ptr, d_pay_in.ptr, d_out.ptr,
                                                d_pay_out.ptr, n, ws.ptr, ws_bytes,
                                                launch.handle))
    ex.synchronize()
    np.testing.assert_array_equal(d_out.to_host_vec(), rows)
    np.testing.assert_array_equal(d_pay_out.to_host_vec(), pay)


def test_radix_many_tiles_and_groups(ex):
    """2^22 rows of arity 2 (512 tiles, 32 look-back groups per pass), small
    interned ids in the first column and full-range ids in the second."""
    n = 1 << 22
    rows = np.empty((n, 2), dtype=np.uint32)
    rows[:, 0] = (workloads.hash_range(61, n) % np.uint64(5000)).astype(np.uint32)
    rows[:, 1] = (workloads.hash_range(62, n) >> np.uint64(32)).astype(np.uint32)
    _check(ex, rows, np.arange(n, dtype=np.uint64))


def test_repeated_sorts_reuse_workspace(ex):
    """Back-to-back sorts of different inputs on one workspace (the look-back
    buffers and bins are re-initialised by each call)."""
    from rccl_amd import _abi

    n, arity = 150_001, 4
    ws_bytes = _abi.workspace_bytes("rccl_hip_record_sort_workspace_bytes", arity, 8, n)
    ws = DeviceBuffer.bytes(ws_bytes)
    launch = ex.launch()
    for seed, distinct in ((1, 3), (2, None), (3, 1000)):
        rows = _random_rows(arity, n, seed, distinct=distinct)
        pay = workloads.hash_range(seed + 10, n)
        exp_rows, exp_pay = oracle.record_sort(rows, pay)
        d_rows = rs.RowBuffer.from_host(rows)
        d_pay = DeviceBuffer.from_host(pay)
        _abi.check(_abi.load().rccl_hip_record_sort(arity, 8, d_rows.ptr, d_pay.ptr, d_rows.ptr,
                                                    d_pay.ptr, n, ws.ptr, ws_bytes,
                                                    launch.handle))
        ex.synchronize()
        np.testing.assert_array_equal(d_rows.to_host_vec(), exp_rows)
        np.testing.assert_array_equal(d_pay.to_host_vec(), exp_pay)
