"""GPU parity tests for set operations over unmaterialised arithmetic ranges.

Cases follow rccl-thrust/examples/set_operations_tests.rs:626-661 (the
counting-range difference, and the 2^30..2^33 magnitudes whose result is
fixed in closed form); the rest compare with the CPU oracle's set operation
on the ranges materialised on the host.
"""
import numpy as np
import pytest

import oracle
from rccl_amd import cub, thrust
from rccl_amd.device import DeviceBuffer

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("tile_order")]

OPS = ["union", "intersection", "difference", "symmetric_difference"]
INT_KINDS = {"u8": np.uint8, "i8": np.int8, "u16": np.uint16, "i16": np.int16,
             "u32": np.uint32, "i32": np.int32, "u64": np.uint64, "i64": np.int64}


@pytest.fixture(scope="module")
def exec_(launch):
    return thrust.Execution(launch)


def _run(exec_, op, first, second, descending=False, capacity=None):
    order = thrust.descending if descending else thrust.ascending
    cap = first.len() + second.len() if capacity is None else capacity
    out_k = DeviceBuffer.zeroed(first.dtype, cap)
    n = getattr(first, f"{op}_by")(second, order).write_into(thrust.view_mut(out_k), exec_)
    return out_k.to_host_vec(), n


def test_counting_difference(exec_):
    """set_operations_tests.rs:626-634: [0, 10001) minus [0, 10000) = [10000]."""
    first = thrust.arithmetic_range(np.int64(0), np.int64(1), 10_001)
    second = thrust.arithmetic_range(np.int64(0), np.int64(1), 10_000)
    out = DeviceBuffer.zeroed(np.int64, 1)
    n = first.difference(second).write_into(thrust.view_mut(out), exec_)
    assert n == 1
    assert out.to_host_vec().tolist() == [10_000]


@pytest.mark.parametrize("magnitude", [30, 31, 32, 33])
def test_wide_counting_ranges(exec_, magnitude):
    """set_operations_tests.rs:636-661: ranges past 2^31 items (the reference's
    wide-index path), into a one-item output."""
    count = 1 << magnitude
    out = DeviceBuffer.zeroed(np.int64, 1)
    first = thrust.arithmetic_range(np.int64(0), np.int64(1), count + 1)
    second = thrust.arithmetic_range(np.int64(0), np.int64(1), count)
    assert first.difference(second).write_into(thrust.view_mut(out), exec_) == 1
    assert out.to_host_vec().tolist() == [count]
    second = thrust.arithmetic_range(np.int64(count), np.int64(1), count)
    assert first.intersection(second).write_into(thrust.view_mut(out), exec_) == 1
    assert out.to_host_vec().tolist() == [count]


def _ranges(kind, descending, seed):
    """Two sorted, overlapping, non-wrapping ranges of `kind` with different
    steps (so that some items coincide and some do not)."""
    dt = np.dtype(INT_KINDS[kind])
    info = np.iinfo(dt)
    rng = np.random.default_rng(seed)
    span = min(int(info.max) - int(info.min), 1 << 40)
    n_max = min(int(info.max) + 1, 50_000)  # indices must fit the key type
    out = []
    for _ in range(2):
        step = int(rng.integers(1, 4))
        n = int(rng.integers(n_max // 2, n_max))
        n = max(1, min(n, span // step))
        lo = int(info.min) + int(rng.integers(0, max(1, span - step * n)))
        lo = min(lo, int(info.max) - step * (n - 1))
        if descending:
            start, stp = lo + step * (n - 1), -step
        else:
            start, stp = lo, step
        out.append(thrust.arithmetic_range(np.array(start).astype(dt), np.array(stp).astype(dt),
                                           n))
    return out


@pytest.mark.parametrize("kind", list(INT_KINDS))
@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("descending", [False, True])
def test_arithmetic_vs_oracle(exec_, kind, op, descending):
    first, second = _ranges(kind, descending, sum(map(ord, kind + op)) * 2 + int(descending))
    a, b = first.to_host_vec(), second.to_host_vec()
    assert np.all(a[1:] < a[:-1]) if descending else np.all(a[1:] > a[:-1])
    expected = oracle.set_op(op, kind, a, b, descending=descending)
    got, n = _run(exec_, op, first, second, descending)
    assert n == len(expected)
    assert np.array_equal(got[:n], expected)


def test_overlapping_shifted_ranges(exec_):
    """A wide step-3 range against a step-2 range starting inside it: the
    intersection is the multiples of 6 in the overlap."""
    first = thrust.arithmetic_range(np.uint32(0), np.uint32(3), 1_000_003)
    second = thrust.arithmetic_range(np.uint32(1_000_000), np.uint32(2), 2_000_001)
    a, b = first.to_host_vec(), second.to_host_vec()
    for op in OPS:
        expected = oracle.set_op(op, "u32", a, b)
        got, n = _run(exec_, op, first, second)
        assert n == len(expected), op
        assert np.array_equal(got[:n], expected), op
    inter, n = _run(exec_, "intersection", first, second)
    assert np.all(inter[:n] % 6 == 0) and n == len(range(1_000_002, 3_000_007, 6))


def test_wrapping_arithmetic_u8(exec_):
    """Items are computed in the key's wrapping arithmetic: start 255, step
    255 (= -1 mod 256) counts down from 255 (descending order)."""
    first = thrust.arithmetic_range(np.uint8(255), np.uint8(255), 256)
    second = thrust.arithmetic_range(np.uint8(200), np.uint8(254), 50)  # 200, 198, ...
    a, b = first.to_host_vec(), second.to_host_vec()
    assert a[0] == 255 and a[-1] == 0 and b[-1] == 102
    for op in OPS:
        expected = oracle.set_op(op, "u8", a, b, descending=True)
        got, n = _run(exec_, op, first, second, descending=True)
        assert n == len(expected), op
        assert np.array_equal(got[:n], expected), op


def test_count_only_and_capacity(exec_):
    launch = exec_.launch()
    first = cub.arithmetic_range(np.int32(-5000), np.int32(1), 20_000)
    second = cub.arithmetic_range(np.int32(0), np.int32(7), 9_000)
    a, b = first.to_host_vec(), second.to_host_vec()
    expected = oracle.set_op("union", "i32", a, b)
    ws = cub.device_set_workspace(launch, "union", np.int32, first.len(), second.len())
    cub.device_set_arithmetic(launch, "union", first, second, ws)
    assert ws.count() == len(expected)
    out = DeviceBuffer.zeroed(np.int32, 1000)
    cub.device_set_arithmetic(launch, "union", first, second, ws, out)
    assert ws.count() == len(expected)
    assert np.array_equal(out.to_host_vec(), expected[:1000])


def test_index_must_fit_key(exec_):
    first = thrust.arithmetic_range(np.int8(0), np.int8(1), 129)  # index 128 is not an i8
    second = thrust.arithmetic_range(np.int8(0), np.int8(1), 10)
    out = DeviceBuffer.zeroed(np.int8, 200)
    with pytest.raises(cub.DeviceAlgorithmError, match="first arithmetic range index"):
        first.union(second).write_into(thrust.view_mut(out), exec_)
    ok = thrust.arithmetic_range(np.int8(-128), np.int8(1), 128)
    assert ok.union(second).write_into(thrust.view_mut(out), exec_) == 138  # -128..-1, 0..9
