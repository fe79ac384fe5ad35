"""GPU parity tests for the four sorted multiset operations through the C ABI.

Literal cases and test families follow the reference's own set tests
(rccl-thrust/examples/set_operations.rs:23-96 and
rccl-thrust/examples/set_operations_tests.rs:307-627); every other output is
compared with the CPU oracle, which restates that file's `host_set_by`
(:40-104), on the same seeded input.
"""
import numpy as np
import pytest

import oracle
from rccl_amd import cub, thrust, workloads
from rccl_amd.device import DeviceBuffer

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("tile_order")]

OPS = ["union", "intersection", "difference", "symmetric_difference"]
DTYPES = {"u8": np.uint8, "i8": np.int8, "u16": np.uint16, "i16": np.int16, "u32": np.uint32,
          "i32": np.int32, "f32": np.float32, "u64": np.uint64, "i64": np.int64,
          "f64": np.float64}


@pytest.fixture(scope="module")
def exec_(launch):
    return thrust.Execution(launch)


def _view(host):
    return thrust.view(DeviceBuffer.from_host(host))


def _run(exec_, op, a, b, av=None, bv=None, descending=False, capacity=None):
    """Run `op` through the Thrust mirror; returns (keys, values|None, count)."""
    order = thrust.descending if descending else thrust.ascending
    first, second = _view(a), _view(b)
    if av is not None:
        first = first.with_values(DeviceBuffer.from_host(av))
        second = second.with_values(DeviceBuffer.from_host(bv)) if bv is not None else second
    cap = a.size + b.size if capacity is None else capacity
    out_k = DeviceBuffer.zeroed(a.dtype, cap)
    out = thrust.view_mut(out_k)
    out_v = None
    if av is not None:
        out_v = DeviceBuffer.zeroed(av.dtype, cap)
        out = out.with_values(out_v)
    n = getattr(first, f"{op}_by")(second, order).write_into(out, exec_)
    keys = out_k.to_host_vec()
    vals = None if out_v is None else out_v.to_host_vec()
    return keys, vals, n


def _bits(a):
    return a.view(np.dtype(f"u{a.dtype.itemsize}"))


# ---------------------------------------------------------------------------
# Literal cases.
# ---------------------------------------------------------------------------
def test_set_operations_example(exec_):
    # rccl-thrust/examples/set_operations.rs:23-96
    a = np.array([0, 2, 4, 5, 6, 8, 9], np.int32)
    b = np.array([0, 1, 2, 3, 5, 7, 8], np.int32)
    want = {"union": [0, 1, 2, 3, 4, 5, 6, 7, 8, 9], "intersection": [0, 2, 5, 8],
            "difference": [4, 6, 9], "symmetric_difference": [1, 3, 4, 6, 7, 9]}
    for op, w in want.items():
        k, _, n = _run(exec_, op, a, b)
        assert k[:n].tolist() == w, op
    assert _view(a).intersection(_view(b)).count(exec_) == 4
    av = np.array([10, 20, 40, 50, 60, 80, 90], np.int32)
    bv = np.array([100, 110, 120, 130, 150, 170, 180], np.int32)
    k, v, n = _run(exec_, "union", a, b, av, bv)
    assert k[:n].tolist() == [0, 1, 2, 3, 4, 5, 6, 7, 8, 9]
    assert v[:n].tolist() == [10, 110, 20, 130, 40, 50, 60, 170, 80, 90]


def test_set_multiset_literals(exec_):
    # rccl-thrust/examples/set_operations_tests.rs:314-489
    k, _, n = _run(exec_, "union", np.array([0, 2, 2], np.int32), np.array([0, 2, 2, 2, 3], np.int32))
    assert k[:n].tolist() == [0, 2, 2, 2, 3]
    a = np.array([0, 2, 4, 6], np.int32)
    b = np.array([0, 3, 3, 4, 7], np.int32)
    for op, w in {"intersection": [0, 4], "difference": [2, 6],
                  "symmetric_difference": [2, 3, 3, 6, 7]}.items():
        k, _, n = _run(exec_, op, a, b)
        assert k[:n].tolist() == w, op
    da, db = a[::-1].copy(), b[::-1].copy()
    for op, w in {"union": [7, 6, 4, 3, 3, 2, 0], "intersection": [4, 0], "difference": [6, 2],
                  "symmetric_difference": [7, 6, 3, 3, 2]}.items():
        k, _, n = _run(exec_, op, da, db, descending=True)
        assert k[:n].tolist() == w, ("desc", op)
    av = np.array([10, 12, 14, 16], np.int32)
    bv = np.array([20, 23, 23, 24, 27], np.int32)
    for op, wk, wv in [("union", [0, 2, 3, 3, 4, 6, 7], [10, 12, 23, 23, 14, 16, 27]),
                       ("intersection", [0, 4], [10, 14]), ("difference", [2, 6], [12, 16]),
                       ("symmetric_difference", [2, 3, 3, 6, 7], [12, 23, 23, 16, 27])]:
        k, v, n = _run(exec_, op, a, b, av, bv)
        assert k[:n].tolist() == wk and v[:n].tolist() == wv, op
    dav = np.array([16, 14, 12, 10], np.int32)
    dbv = np.array([27, 24, 23, 33, 20], np.int32)
    for op, wk, wv in [("union", [7, 6, 4, 3, 3, 2, 0], [27, 16, 14, 23, 33, 12, 10]),
                       ("intersection", [4, 0], [14, 10]), ("difference", [6, 2], [16, 12]),
                       ("symmetric_difference", [7, 6, 3, 3, 2], [27, 16, 23, 33, 12])]:
        k, v, n = _run(exec_, op, da, db, dav, dbv, descending=True)
        assert k[:n].tolist() == wk and v[:n].tolist() == wv, ("desc", op)


def test_set_multi_tile_lookback(exec_):
    # rccl-thrust/examples/set_operations_tests.rs:491-537
    n = 25_000
    evens = (np.arange(n) * 2).astype(np.int32)
    odds = (np.arange(n) * 2 + 1).astype(np.int32)
    k, _, m = _run(exec_, "union", evens, odds)
    assert m == 2 * n and np.array_equal(k[:m], np.arange(2 * n, dtype=np.int32))
    assert _run(exec_, "intersection", evens, odds)[2] == 0
    assert _view(evens).union(_view(odds)).count(exec_) == 2 * n
    assert _view(evens).intersection(_view(odds)).count(exec_) == 0
    k, _, m = _run(exec_, "union", evens, evens.copy())
    assert m == n and np.array_equal(k[:m], evens)
    assert _run(exec_, "difference", evens, evens.copy())[2] == 0


def test_set_low_cardinality_family(exec_):
    # rccl-thrust/examples/set_operations_tests.rs:542-590
    first = np.sort(((np.arange(4097) * 37 + 11) % 13 - 6).astype(np.int32))
    second_all = np.sort(((np.arange(8194) * 29 + 7) % 13 - 6).astype(np.int32))
    for second_len in [0, 1, 2048, 4097, 4098, 8194]:
        second = second_all[:second_len]
        for op in OPS:
            k, _, n = _run(exec_, op, first, second)
            want = oracle.set_op(op, "i32", first, second)
            assert n == want.size and np.array_equal(k[:n], want), (op, second_len)


def test_set_empty(exec_):
    # rccl-thrust/examples/set_operations_tests.rs:592-600
    e = np.zeros(0, np.int32)
    assert _view(e).union(_view(e)).write_into(thrust.view_mut(DeviceBuffer.zeroed(np.int32, 0)),
                                               exec_) == 0


def _by_key_inputs(kind, descending, n_first, n_second):
    dt = np.dtype(DTYPES[kind])
    i1 = np.arange(n_first)
    i2 = np.arange(n_second)
    fk, fv = ((i1 * 37 + 11) % 17).astype(dt), ((i1 * 5 + 1) % 97).astype(dt)
    sk, sv = ((i2 * 29 + 7) % 17).astype(dt), ((i2 * 11 + 3) % 97).astype(dt)
    # Rust's stable sort by key (reversed comparator for descending).
    o1 = np.argsort(-fk.astype(np.float64) if descending else fk, kind="stable")
    o2 = np.argsort(-sk.astype(np.float64) if descending else sk, kind="stable")
    return fk[o1], fv[o1], sk[o2], sv[o2]


@pytest.mark.parametrize("kind", ["i8", "u8", "i16", "u16", "i32", "u32", "f32", "f64"])
def test_set_by_key_family(exec_, kind):
    # rccl-thrust/examples/set_operations_tests.rs:203-305 (and the key_value
    # record family :125-201, whose records order by key with the value as
    # payload, which is the by-key form)
    for descending in (False, True):
        for n_second in (4097, 8194):
            fk, fv, sk, sv = _by_key_inputs(kind, descending, 4097, n_second)
            for op in OPS:
                # Intersection takes the second range as keys only (:286-288).
                bv = None if op == "intersection" else sv
                k, v, n = _run(exec_, op, fk, sk, fv, bv, descending)
                wk, wv = oracle.set_op(op, kind, fk, sk, fv, sv, descending)
                assert n == wk.size, (kind, op, descending, n_second)
                assert np.array_equal(_bits(k[:n]), _bits(wk)), (kind, op, descending)
                assert np.array_equal(_bits(v[:n]), _bits(wv)), (kind, op, descending)


# ---------------------------------------------------------------------------
# Oracle parity: kinds, widths, counts, capacity, C5 shape.
# ---------------------------------------------------------------------------
def _multiset(kind, n, seed, distinct, descending):
    raw = workloads.hash_range(seed, n) % np.uint64(distinct)
    dt = np.dtype(DTYPES[kind])
    keys = raw.astype(np.int64)
    if dt.kind != "u":
        keys -= distinct // 2
    keys = np.sort(keys.astype(dt), kind="stable")
    return keys[::-1].copy() if descending else keys


@pytest.mark.parametrize("kind", ["u8", "i16", "u32", "i32", "f32", "u64", "i64", "f64"])
@pytest.mark.parametrize("op", OPS)
def test_set_keys_vs_oracle(exec_, kind, op):
    for idx, (na, nb, distinct) in enumerate([(1, 0, 5), (0, 3, 5), (1000, 1000, 50),
                                              (20_000, 5_000, 1000), (70_000, 90_000, 120),
                                              (200_000, 150_000, 1 << 20)]):
        distinct = min(distinct, 250) if kind in ("u8", "i8") else distinct
        for descending in (False, True):
            a = _multiset(kind, na, 10 + idx, distinct, descending)
            b = _multiset(kind, nb, 20 + idx, distinct, descending)
            k, _, n = _run(exec_, op, a, b, descending=descending)
            want = oracle.set_op(op, kind, a, b, descending=descending)
            assert n == want.size, (kind, op, na, nb, descending)
            assert np.array_equal(_bits(k[:n]), _bits(want)), (kind, op, na, nb, descending)
            cnt = getattr(_view(a), f"{op}_by")(
                _view(b), thrust.descending if descending else thrust.ascending).count(exec_)
            assert cnt == want.size


@pytest.mark.parametrize("width", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("op", OPS)
def test_set_pairs_widths(exec_, width, op):
    for idx, (na, nb, distinct) in enumerate([(3000, 5000, 40), (60_000, 40_000, 5000)]):
        a = _multiset("u64", na, 30 + idx, distinct, False)
        b = _multiset("u64", nb, 40 + idx, distinct, False)
        if width == 16:
            av = workloads.hash_range(50 + idx, 2 * na).view(np.dtype((np.void, 16)))
            bv = workloads.hash_range(60 + idx, 2 * nb).view(np.dtype((np.void, 16)))
        else:
            dt = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[width]
            av = (workloads.hash_range(50 + idx, na) >> np.uint64(64 - 8 * width)).astype(dt)
            bv = (workloads.hash_range(60 + idx, nb) >> np.uint64(64 - 8 * width)).astype(dt)
        k, v, n = _run(exec_, op, a, b, av, bv)
        wk, wv = oracle.set_op(op, "u64", a, b, av, bv)
        assert n == wk.size
        assert np.array_equal(k[:n], wk)
        assert v[:n].tobytes() == wv.tobytes()


def test_set_output_capacity(exec_):
    """A destination smaller than the result: the full length is counted and
    only the first `capacity` items are written (the reference's own tests
    size outputs to the expected result, set_operations_tests.rs:620-660)."""
    a = np.arange(10_001, dtype=np.int64)
    b = np.arange(10_000, dtype=np.int64)
    k, _, n = _run(exec_, "difference", a, b, capacity=1)
    assert n == 1 and k.tolist() == [10_000]
    a = np.arange(100_000, dtype=np.int64)
    b = np.arange(100_000, dtype=np.int64) * 2
    k, _, n = _run(exec_, "union", a, b, capacity=777)
    want = oracle.set_op("union", "i64", a, b)
    assert n == want.size and np.array_equal(k, want[:777])


def test_set_c5_scaled(exec_):
    """C5 shape (sorted u64 multisets, shared pool, duplicated runs) at 2^20
    per side: every operation bit-exact with the oracle."""
    a, b = workloads.c5_inputs(1 << 20)
    for op in OPS:
        k, _, n = _run(exec_, op, a, b)
        want = oracle.set_op(op, "u64", a, b)
        assert n == want.size and np.array_equal(k[:n], want), op


def _sampled_set_inputs(kind, descending):
    """Sorted multisets of at least 512 partition tiles (the sampled
    partition), with the shapes that stress the sample bracket and the
    balanced path's equal-key runs: heavy duplicates (runs spanning many
    tiles), uniform keys, one side far shorter, all keys equal, and disjoint
    ranges either way round."""
    dt = np.dtype({"u8": np.uint8, "u32": np.uint32, "i64": np.int64}[kind])
    n = (1 << 22) + 5
    info = np.iinfo(dt)

    def rnd(size, seed, distinct=None):
        raw = workloads.hash_range(seed, size)
        if distinct is not None:
            raw = raw % np.uint64(distinct)
        v = raw.astype(dt) if dt.kind == "u" else (raw >> np.uint64(1)).astype(dt)
        s = np.sort(v, kind="stable")
        return s[::-1].copy() if descending else s

    yield "dups", rnd(n, 61, 37), rnd(n - 9, 62, 37)
    yield "uniform", rnd(n, 63), rnd(n + 2047, 64)
    yield "short_b", rnd(2 * n, 65, 1000), rnd(3001, 66, 1000)
    yield "all_equal", np.full(n, 5, dt), np.full(n + 3, 5, dt)
    lo, hi = np.full(n, info.min, dt), np.full(n + 7, info.max, dt)
    first, second = (hi, lo) if descending else (lo, hi)
    yield "disjoint", first, second
    yield "disjoint_reversed", second, first


@pytest.mark.parametrize("kind", ["u8", "u32", "i64"])
@pytest.mark.parametrize("descending", [False, True])
def test_set_sampled_partition_vs_oracle(exec_, kind, descending):
    for idx, (name, a, b) in enumerate(_sampled_set_inputs(kind, descending)):
        for op in OPS:
            if idx == 1 and op in ("union", "symmetric_difference"):
                av = np.arange(a.size, dtype=np.uint32)
                bv = np.arange(b.size, dtype=np.uint32) | np.uint32(1 << 31)
                k, v, n = _run(exec_, op, a, b, av, bv, descending)
                wk, wv = oracle.set_op(op, kind, a, b, av, bv, descending)
                assert n == wk.size and np.array_equal(v[:n], wv), (kind, name, op)
            else:
                k, _, n = _run(exec_, op, a, b, descending=descending)
                wk = oracle.set_op(op, kind, a, b, descending=descending)
            assert n == wk.size and np.array_equal(k[:n], wk), (kind, name, op, descending)
