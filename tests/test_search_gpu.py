"""GPU tests for the vectorized lower_bound / upper_bound.

The reference exports no bound search (CCCL_RUST_CAPABILITY_CHECKLIST.md:107
lists thrust::lower_bound as missing), so there is no reference vector to
match. The results are fixed by the definition instead: on a sorted haystack,
lower_bound(x) is the number of items before x (h < x) and upper_bound(x) the
number not after it (!(x < h)). Tests check that count directly on small
inputs and numpy.searchsorted (the textbook routine) on large ones.
"""
import numpy as np
import pytest

from rccl_amd import record_sort as rs
from rccl_amd import thrust, workloads
from rccl_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu

NP = {"u8": np.uint8, "i8": np.int8, "u16": np.uint16, "i16": np.int16, "u32": np.uint32,
      "i32": np.int32, "f32": np.float32, "u64": np.uint64, "i64": np.int64, "f64": np.float64}


@pytest.fixture(scope="module")
def ex(launch):
    return thrust.Execution(launch)


def _search(ex, hay, needles, upper=False, descending=False):
    rows = hay.ndim == 2
    h = rs.RowBuffer.from_host(hay) if rows else DeviceBuffer.from_host(hay)
    q = rs.RowBuffer.from_host(needles) if rows else DeviceBuffer.from_host(needles)
    out = DeviceBuffer.from_host(np.full(len(needles), 2**64 - 1, dtype=np.uint64))
    order = thrust.descending if descending else thrust.ascending
    (thrust.upper_bound if upper else thrust.lower_bound)(ex, h, q, out, order)
    return out.to_host_vec()


def _values(kind, n, seed, distinct):
    raw = workloads.hash_range(seed, n) % np.uint64(distinct)
    dt = np.dtype(NP[kind])
    v = raw.astype(np.int64) - (distinct // 2 if dt.kind != "u" else 0)
    if dt.kind == "f":
        return (v.astype(np.float64) * 0.5).astype(dt)
    return v.astype(dt)


@pytest.mark.parametrize("n", [0, 1, 2, 3, 7, 64, 100])
def test_definition_small(ex, n):
    """Brute force: the count of haystack items before each needle."""
    hay = np.sort(_values("i32", n, 1, 20))
    needles = np.arange(-12, 13, dtype=np.int32)
    lo = _search(ex, hay, needles)
    up = _search(ex, hay, needles, upper=True)
    assert lo.tolist() == [int(np.sum(hay < x)) for x in needles]
    assert up.tolist() == [int(np.sum(hay <= x)) for x in needles]


@pytest.mark.parametrize("kind", list(NP))
def test_kinds_vs_searchsorted(ex, kind):
    n = 1_000_003
    hay = np.sort(_values(kind, n, 3 + len(kind), 500_000))
    needles = _values(kind, 300_001, 9, 520_000)
    assert np.array_equal(_search(ex, hay, needles), np.searchsorted(hay, needles, "left"))
    assert np.array_equal(_search(ex, hay, needles, upper=True),
                          np.searchsorted(hay, needles, "right"))


@pytest.mark.parametrize("kind", ["u32", "i64", "f32"])
def test_descending(ex, kind):
    """Under the reversed order, items before x are those greater than x."""
    hay = np.sort(_values(kind, 200_003, 21, 90_000))[::-1].copy()
    needles = _values(kind, 50_000, 22, 100_000)
    lo = _search(ex, hay, needles, descending=True)
    up = _search(ex, hay, needles, upper=True, descending=True)
    rev = hay[::-1]
    assert np.array_equal(lo, len(hay) - np.searchsorted(rev, needles, "right"))
    assert np.array_equal(up, len(hay) - np.searchsorted(rev, needles, "left"))


@pytest.mark.parametrize("arity", [2, 3, 4, 5, 6])
def test_rows(ex, arity):
    """Lexicographic rows: compare with searchsorted over the rows viewed as
    big-endian-ordered structured records."""
    n = 100_003
    rows = (workloads.hash_range(40 + arity, n * arity) % np.uint64(7)).astype(
        np.uint32).reshape(n, arity)
    hay = rows[np.lexsort(rows.T[::-1])]
    needles = (workloads.hash_range(50 + arity, 5000 * arity) % np.uint64(8)).astype(
        np.uint32).reshape(5000, arity)
    rec = np.dtype([(f"c{i}", np.uint32) for i in range(arity)])
    h_rec = np.ascontiguousarray(hay).view(rec).ravel()
    q_rec = np.ascontiguousarray(needles).view(rec).ravel()
    assert np.array_equal(_search(ex, hay, needles), np.searchsorted(h_rec, q_rec, "left"))
    assert np.array_equal(_search(ex, hay, needles, upper=True),
                          np.searchsorted(h_rec, q_rec, "right"))


def test_large_haystack_and_extremes(ex):
    """2^26 sorted u32 haystack (the per-level bracketing crosses many sample
    spans), needles below, inside and above the range, and equal runs."""
    n = 1 << 26
    hay = np.sort((workloads.hash_range(77, n) >> np.uint64(40)).astype(np.uint32))
    needles = np.concatenate([np.array([0, 1, 2**32 - 1, hay[0], hay[-1], hay[n // 2]],
                                       dtype=np.uint32),
                              (workloads.hash_range(78, 1 << 20) >> np.uint64(40)).astype(
                                  np.uint32)])
    assert np.array_equal(_search(ex, hay, needles), np.searchsorted(hay, needles, "left"))
    assert np.array_equal(_search(ex, hay, needles, upper=True),
                          np.searchsorted(hay, needles, "right"))


def test_output_capacity(ex):
    hay = DeviceBuffer.from_host(np.arange(10, dtype=np.uint32))
    q = DeviceBuffer.from_host(np.arange(5, dtype=np.uint32))
    with pytest.raises(thrust.DeviceAlgorithmError, match="bound-search output"):
        thrust.lower_bound(ex, hay, q, DeviceBuffer.zeroed(np.uint64, 4))


@pytest.mark.parametrize("kind", ["u8", "i16", "u32", "f64"])
def test_index_and_direct_paths(ex, kind):
    """A large haystack: many needles search through the per-call chunk index,
    a few search the haystack directly; both agree with searchsorted, for
    needles drawn from the values, haystack items at and around chunk
    boundaries (every chunk is 128 bytes), and the extremes."""
    n = (1 << 22) + 5
    distinct = 256 if kind == "u8" else 1 << 20
    hay = np.sort(_values(kind, n, 31, distinct))
    chunk = 128 // hay.dtype.itemsize
    edges = np.arange(chunk - 1, n, chunk * 97)
    for m in (300_001, 1_000):
        needles = np.concatenate([hay[[0, n - 1]], hay[edges], hay[np.minimum(edges + 1, n - 1)],
                                  _values(kind, m, 32, distinct + 7)])[:m]
        assert np.array_equal(_search(ex, hay, needles), np.searchsorted(hay, needles, "left"))
        assert np.array_equal(_search(ex, hay, needles, upper=True),
                              np.searchsorted(hay, needles, "right"))


@pytest.mark.parametrize("kind", ["u32", "f64"])
def test_unaligned_haystack(ex, kind):
    """A haystack that starts one item past a 16-byte boundary: the index
    levels are still read a line at a time, the haystack chunk by binary
    search."""
    n = (1 << 21) + 3
    hay = np.sort(_values(kind, n, 41, 1 << 19))
    padded = DeviceBuffer.from_host(np.concatenate([hay[:1], hay]))
    h = DeviceBuffer(padded.tensor[1:], hay.dtype, n)
    assert h.ptr % 16 != 0
    needles = np.concatenate([hay[[0, n - 1]], _values(kind, 200_000, 42, (1 << 19) + 5)])
    for upper, side in ((False, "left"), (True, "right")):
        out = DeviceBuffer.from_host(np.full(len(needles), 2**64 - 1, dtype=np.uint64))
        (thrust.upper_bound if upper else thrust.lower_bound)(
            ex, h, DeviceBuffer.from_host(needles), out)
        assert np.array_equal(out.to_host_vec(), np.searchsorted(hay, needles, side))
