"""GPU parity tests for the adjacent-run compactions (unique, reduce-by-key).

Literal cases come from the reference's examples (rccl-thrust/examples/
compaction.rs, grouped_reduction.rs, also golden vectors); the families and
random cases compare every output bit-for-bit with the CPU oracle
(oracle_unique / oracle_reduce_by_key) on the same input.
"""
import json
import os

import numpy as np
import pytest

import oracle
from rccl_amd import record_sort as rs
from rccl_amd import thrust, workloads
from rccl_amd.device import DeviceBuffer

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("tile_order")]

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.json")
NP = {"u8": np.uint8, "i8": np.int8, "u16": np.uint16, "i16": np.int16, "u32": np.uint32,
      "i32": np.int32, "f32": np.float32, "u64": np.uint64, "i64": np.int64, "f64": np.float64}
OPERATORS = {"natural_bag_add": thrust.NaturalBagAdd, "boolean_or": thrust.BooleanOr,
             "independent_probability_or": thrust.IndependentProbabilityOr}


@pytest.fixture(scope="module")
def ex(launch):
    return thrust.Execution(launch)


def _dev(a):
    return DeviceBuffer.from_host(a)


def _unique(ex, keys, pays=None):
    """Run unique_copy_by; returns (keys, payloads|None, count)."""
    n = len(keys)
    rows = keys.ndim == 2
    k_in = rs.RowBuffer.from_host(keys) if rows else _dev(keys)
    k_out = rs.RowBuffer.zeroed(keys.shape[1], n) if rows else DeviceBuffer.zeroed(keys.dtype, n)
    count = DeviceBuffer.from_host(np.array([2**64 - 1], dtype=np.uint64))
    if pays is None:
        thrust.unique_copy_by(ex, k_in, k_out, count)
    else:
        p_out = DeviceBuffer.zeroed(pays.dtype, n)
        thrust.unique_copy_by(ex, (k_in, _dev(pays)), (k_out, p_out), count)
    c = int(count.to_host_vec()[0])
    return k_out.to_host_vec()[:c], (None if pays is None else p_out.to_host_vec()[:c]), c


def _reduce(ex, keys, vals, op, pays=None):
    n = len(keys)
    rows = keys.ndim == 2
    k_in = rs.RowBuffer.from_host(keys) if rows else _dev(keys)
    k_out = rs.RowBuffer.zeroed(keys.shape[1], n) if rows else DeviceBuffer.zeroed(keys.dtype, n)
    v_out = DeviceBuffer.zeroed(vals.dtype, n)
    groups = DeviceBuffer.from_host(np.array([2**64 - 1], dtype=np.uint64))
    if pays is None:
        thrust.reduce_by_key(ex, k_in, _dev(vals), k_out, v_out, groups, thrust.equal,
                             OPERATORS[op])
    else:
        p_out = DeviceBuffer.zeroed(pays.dtype, n)
        thrust.reduce_by_key(ex, (k_in, _dev(pays)), _dev(vals), (k_out, p_out), v_out, groups,
                             thrust.equal, OPERATORS[op])
    c = int(groups.to_host_vec()[0])
    return (k_out.to_host_vec()[:c], None if pays is None else p_out.to_host_vec()[:c],
            v_out.to_host_vec()[:c], c)


def _bits(a):
    return a.view(np.dtype(f"u{a.dtype.itemsize}"))


def test_golden_vectors(ex):
    cases = [c for c in json.load(open(GOLDEN))["cases"] if c["op"] in ("unique", "reduce_by_key")]
    assert len(cases) >= 5
    for c in cases:
        keys = np.array(c["keys"], dtype=NP[c["kind"]])
        pays = None
        if "payloads" in c:
            pays = np.array(c["payloads"], dtype=NP[c["payload_dtype"]])
        if c["op"] == "unique":
            k, p, n = _unique(ex, keys, pays)
            assert k.tolist() == c["expected_keys"], c["id"]
            assert p.tolist() == c["expected_payloads"], c["id"]
            continue
        if "values" in c:
            vals = np.array(c["values"], dtype=OPERATORS[c["group_op"]].dtype)
        else:
            vals = np.array(c["values_f64_bits"], dtype=np.uint64).view(np.float64)
        k, p, v, n = _reduce(ex, keys, vals, c["group_op"], pays)
        assert k.tolist() == c["expected_keys"], c["id"]
        if "expected_values_f64_bits" in c:
            assert v.view(np.uint64).tolist() == c["expected_values_f64_bits"], c["id"]
        else:
            assert v.astype(np.uint64).tolist() == c["expected_values"], c["id"]
        if "expected_payloads" in c:
            assert p.tolist() == c["expected_payloads"], c["id"]


@pytest.mark.parametrize("n", [0, 1, 31, 32, 33, 255, 256, 257, 513])
def test_unique_boundaries(ex, n):
    """examples/compaction.rs:117-146: input[i] = i / 3."""
    keys = (np.arange(n) // 3).astype(np.uint32)
    k, _, c = _unique(ex, keys)
    assert np.array_equal(k, oracle.unique(keys, "u32"))


@pytest.mark.parametrize("n", [0, 1, 31, 32, 33, 255, 256, 257, 513, 65_537])
@pytest.mark.parametrize("pattern", [0, 1, 2])
def test_reduce_u64_boundaries(ex, n, pattern):
    """examples/grouped_reduction.rs:31-82 (one run, all distinct, runs of 3
    repeating over 11 keys; values with u64::MAX every 17th)."""
    i = np.arange(n)
    keys = {0: np.full(n, 7), 1: i, 2: (i // 3) % 11}[pattern].astype(np.uint32)
    vals = np.where(i % 17 == 0, np.uint64(2**64 - 1), (i % 13 + 1).astype(np.uint64))
    vals = vals.astype(np.uint64)
    k, _, v, c = _reduce(ex, keys, vals, "natural_bag_add")
    ek, ev = oracle.reduce_by_key(keys, vals, "natural_bag_add", "u32")
    assert c == len(ek)
    assert np.array_equal(k, ek) and np.array_equal(v, ev)


KINDS = ["u8", "i8", "u16", "i16", "u32", "i32", "f32", "u64", "i64", "f64"]


def _sorted_keys(kind, n, seed, distinct):
    raw = workloads.hash_range(seed, n) % np.uint64(distinct)
    dt = np.dtype(NP[kind])
    keys = np.sort(raw).astype(np.int64)
    if dt.kind == "f":
        return (keys.astype(np.float64) * 0.25 - 3.0).astype(dt)
    return keys.astype(dt)


@pytest.mark.parametrize("kind", KINDS)
def test_unique_kinds_with_payloads(ex, kind):
    n = 100_003
    keys = _sorted_keys(kind, n, 30 + KINDS.index(kind), distinct=120)
    for pay_dt in (None, np.uint8, np.uint16, np.uint32, np.uint64):
        pays = None if pay_dt is None else (workloads.hash_range(7, n) >> np.uint64(40)).astype(
            pay_dt)
        k, p, c = _unique(ex, keys, pays)
        heads = np.flatnonzero(np.r_[True, keys[1:] != keys[:-1]])
        assert np.array_equal(_bits(k), _bits(oracle.unique(keys, kind)))
        if pays is not None:
            assert np.array_equal(p, pays[heads])


@pytest.mark.parametrize("kind", ["u32", "i64", "f64", "u8"])
@pytest.mark.parametrize("op", list(OPERATORS))
def test_reduce_kinds_and_ops(ex, kind, op):
    n = 200_001
    keys = _sorted_keys(kind, n, 50 + KINDS.index(kind), distinct=3000)
    raw = workloads.hash_range(51, n)
    vals = {"natural_bag_add": raw,
            "boolean_or": (raw & np.uint64(1)).astype(np.uint8),
            "independent_probability_or": (raw >> np.uint64(11)).astype(np.float64) / 2**53}[op]
    for pays in (None, (raw >> np.uint64(32)).astype(np.uint32)):
        k, p, v, c = _reduce(ex, keys, vals, op, pays)
        ek, ev = oracle.reduce_by_key(keys, vals, op, kind)
        assert c == len(ek)
        assert np.array_equal(_bits(k), _bits(ek))
        assert np.array_equal(_bits(v), _bits(ev))  # the left fold is bit-exact
        if pays is not None:
            heads = np.flatnonzero(np.r_[True, keys[1:] != keys[:-1]])
            assert np.array_equal(p, pays[heads])


def test_float_equality_rules(ex):
    """IEEE ==: -0.0 joins a run of +0.0; NaN never joins a run."""
    keys = np.array([0.0, -0.0, np.nan, np.nan, 1.0, 1.0, -np.inf, -np.inf], dtype=np.float32)
    k, _, c = _unique(ex, keys)
    assert np.array_equal(_bits(k), _bits(oracle.unique(keys, "f32")))
    assert c == 5


@pytest.mark.parametrize("arity", [2, 3, 4, 5, 6])
def test_rows_dedup_after_record_sort(ex, arity):
    """The datalog step after a row sort: sort rows with provenance, then
    unique (keep the first provenance) and reduce (fold provenance)."""
    n = 150_001
    rows = (workloads.hash_range(70 + arity, n * arity) % np.uint64(4)).astype(
        np.uint32).reshape(n, arity)
    prov = workloads.hash_range(80 + arity, n)
    srows, sprov = oracle.record_sort(rows, prov)
    k, p, c = _unique(ex, srows, sprov)
    ek = oracle.unique(srows)
    heads = np.flatnonzero(np.r_[True, np.any(srows[1:] != srows[:-1], axis=1)])
    assert np.array_equal(k, ek) and np.array_equal(p, sprov[heads])
    k, _, v, c = _reduce(ex, srows, sprov, "natural_bag_add")
    ek, ev = oracle.reduce_by_key(srows, sprov, "natural_bag_add")
    assert np.array_equal(k, ek) and np.array_equal(v, ev)


def test_long_runs_cross_tiles(ex):
    """Runs much longer than a tile: the fold continues past the tile's end
    in global memory, in index order."""
    n = 300_000
    keys = np.repeat(np.arange(4, dtype=np.int32), [1, 150_000, 149_998, 1])
    vals = (workloads.hash_range(90, n) >> np.uint64(11)).astype(np.float64) / 2**53 * 1e-3
    for op, vv in (("independent_probability_or", vals),
                   ("natural_bag_add", workloads.hash_range(91, n))):
        k, _, v, c = _reduce(ex, keys, vv, op)
        ek, ev = oracle.reduce_by_key(keys, vv, op, "i32")
        assert c == 4 and np.array_equal(k, ek) and np.array_equal(_bits(v), _bits(ev))


def test_unique_by_in_place(ex):
    """examples/compaction.rs:89-114: in place through a scratch range; the
    tail of the values keeps its old contents."""
    keys = np.array([1, 1, 2, 2, 2, 1, 3, 3], dtype=np.uint32)
    prov = np.array([10, 11, 20, 21, 22, 12, 30, 31], dtype=np.uint64)
    dk, dp = _dev(keys), _dev(prov)
    sk, sp = DeviceBuffer.zeroed(np.uint32, 8), DeviceBuffer.zeroed(np.uint64, 8)
    count = DeviceBuffer.zeroed(np.uint64, 1)
    thrust.unique_by(ex, thrust.view(dk).with_values(dp), thrust.view(sk).with_values(sp), count)
    c = int(count.to_host_vec()[0])
    assert c == 4
    assert dk.to_host_vec().tolist() == [1, 2, 1, 3, 2, 1, 3, 3]
    assert dp.to_host_vec().tolist() == [10, 20, 12, 30, 22, 12, 30, 31]


def test_contract_errors(ex):
    """examples/grouped_reduction.rs:226-282 and compaction.rs:208-230."""
    keys = _dev(np.array([1, 1, 2], dtype=np.uint32))
    values = _dev(np.array([1, 2, 3], dtype=np.uint64))
    out_k, out_v = DeviceBuffer.zeroed(np.uint32, 3), DeviceBuffer.zeroed(np.uint64, 3)
    groups = DeviceBuffer.zeroed(np.uint64, 1)
    with pytest.raises(thrust.DeviceAlgorithmError, match="values length"):
        thrust.reduce_by_key(ex, keys, _dev(np.array([1, 2], dtype=np.uint64)), out_k, out_v,
                             groups)
    with pytest.raises(thrust.DeviceAlgorithmError, match="key output"):
        thrust.reduce_by_key(ex, keys, values, DeviceBuffer.zeroed(np.uint32, 2), out_v, groups)
    with pytest.raises(thrust.DeviceAlgorithmError, match="aggregate output"):
        thrust.reduce_by_key(ex, keys, values, out_k, DeviceBuffer.zeroed(np.uint64, 2), groups)
    with pytest.raises(thrust.DeviceAlgorithmError, match="group-count output"):
        thrust.reduce_by_key(ex, keys, values, out_k, out_v, DeviceBuffer.zeroed(np.uint64, 0))
    with pytest.raises(thrust.DeviceAlgorithmError, match="unique-copy output"):
        thrust.unique_copy_by(ex, keys, DeviceBuffer.zeroed(np.uint32, 2), groups)
    with pytest.raises(ValueError):
        thrust.unique_copy_by(ex, keys, out_k, groups, lambda a, b: a == b)
