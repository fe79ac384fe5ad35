"""GPU tests of the Thrust sort surface: sort, sort_unstable, sort_by,
sort_unstable_by on buffers and on with_values(..) key/value ranges.

Vectors are the reference's pinned Thrust examples
(rccl-thrust/examples/sort.rs:16-191 and comparison_sort.rs:10-89). Closures
are classified on the host into the natural order or its reverse (each with
a prebuilt kernel); the reference's custom comparators (evens first, parity
then value, by decade) have no kernel here and must be rejected before any
launch, leaving the input untouched.
"""
import numpy as np
import pytest

from rccl_amd import cub, thrust
from rccl_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu

UPSTREAM = [79, 78, 62, 78, 94, 40, 86, 57, 40, 16, 28, 54, 77, 87, 93, 98]  # sort.rs:16-19
UP_ASC = [16, 28, 40, 40, 54, 57, 62, 77, 78, 78, 79, 86, 87, 93, 94, 98]
UP_DESC = UP_ASC[::-1]
STABLE_IN = [25, 14, 35, 16, 26, 34, 36, 24, 15]  # sort.rs:106-107


def rust_cmp(a, b):
    """`a.cmp(b)` as a closure result."""
    return (a > b) - (a < b)


def rev_cmp(left, right):
    """`|left, right| right.cmp(left)`."""
    return rust_cmp(right, left)


@pytest.fixture(scope="module")
def ex():
    return thrust.Program.load(0).par()


def _buf(values, dt=np.int32):
    return DeviceBuffer.from_host(np.array(values, dtype=dt))


def test_upstream_natural_and_descending(ex):
    # sort.rs:20-34
    b = _buf(UPSTREAM)
    thrust.view_mut(b).sort_unstable(ex)
    assert b.to_host_vec().tolist() == UP_ASC
    b = _buf(UPSTREAM)
    thrust.view_mut(b).sort_unstable_by(ex, rev_cmp)
    assert b.to_host_vec().tolist() == UP_DESC


def test_upstream_pairs_natural_and_descending(ex):
    # sort.rs:51-90: values are original positions, stable among equal keys
    k, v = _buf(UPSTREAM), _buf(range(16))
    thrust.view_mut(k).with_values(thrust.view_mut(v)).sort_unstable(ex)
    assert k.to_host_vec().tolist() == UP_ASC
    assert v.to_host_vec().tolist() == [9, 10, 5, 8, 11, 7, 2, 12, 1, 3, 0, 6, 13, 14, 4, 15]
    k, v = _buf(UPSTREAM), _buf(range(16))
    thrust.view_mut(k).with_values(thrust.view_mut(v)).sort_unstable_by(ex, rev_cmp)
    assert k.to_host_vec().tolist() == UP_DESC
    assert v.to_host_vec().tolist() == [15, 4, 14, 13, 6, 0, 1, 3, 12, 2, 7, 11, 5, 8, 10, 9]


def test_small_simple_cases(ex):
    # sort.rs:92-98, :121-150
    b = _buf([1, 3, 6, 5, 2, 0, 4])
    thrust.view_mut(b).sort_unstable(ex)
    assert b.to_host_vec().tolist() == [0, 1, 2, 3, 4, 5, 6]
    b = _buf([1, 3, 6, 5, 2, 0, 4])
    thrust.view_mut(b).sort_unstable_by(ex, rev_cmp)
    assert b.to_host_vec().tolist() == [6, 5, 4, 3, 2, 1, 0]
    b = _buf([3, 1, 2, 1])
    thrust.view_mut(b).sort(ex)
    assert b.to_host_vec().tolist() == [1, 1, 2, 3]
    k, v = _buf([1, 3, 6, 5, 2, 0, 4]), _buf(range(7))
    thrust.view_mut(k).with_values(thrust.view_mut(v)).sort(ex)
    assert k.to_host_vec().tolist() == [0, 1, 2, 3, 4, 5, 6]
    assert v.to_host_vec().tolist() == [5, 0, 4, 1, 6, 3, 2]
    k, v = _buf([1, 3, 6, 5, 2, 0, 4]), _buf(range(7))
    thrust.view_mut(k).with_values(thrust.view_mut(v)).sort_unstable_by(ex, rev_cmp)
    assert k.to_host_vec().tolist() == [6, 5, 4, 3, 2, 1, 0]
    assert v.to_host_vec().tolist() == [2, 3, 6, 1, 4, 0, 5]
    k, v = _buf([1, 3, 6, 5, 2, 0, 4]), _buf(range(7))
    thrust.view_mut(k).with_values(thrust.view_mut(v)).sort_unstable(ex)
    assert k.to_host_vec().tolist() == [0, 1, 2, 3, 4, 5, 6]
    assert v.to_host_vec().tolist() == [5, 0, 4, 1, 6, 3, 2]


def test_float_pairs_signed_zero(ex):
    # sort.rs:164-191
    keys = np.array([1.25, -0.0, np.inf, -3.5, 0.0, -np.inf], np.float32)
    k, v = DeviceBuffer.from_host(keys), _buf([4, 2, 5, 1, 3, 0])
    thrust.view_mut(k).with_values(thrust.view_mut(v)).sort(ex)
    want = np.array([-np.inf, -3.5, -0.0, 0.0, 1.25, np.inf], np.float32)
    assert k.to_host_vec().view(np.uint32).tolist() == want.view(np.uint32).tolist()
    assert v.to_host_vec().tolist() == [0, 1, 2, 3, 4, 5]


def test_equivalent_closures_lower(ex):
    """Closures written differently from the library's own comparators lower
    to the same kernels (classification by probing, not identity)."""
    b = _buf(UPSTREAM)
    thrust.view_mut(b).sort_by(ex, lambda l, r: -1 if l < r else (1 if l > r else 0))
    assert b.to_host_vec().tolist() == UP_ASC
    b = _buf(UPSTREAM, np.uint64)
    thrust.view_mut(b).sort_by(ex, lambda l, r: (r > l) - (r < l))
    assert b.to_host_vec().tolist() == UP_DESC
    f = np.array([2.5, -0.0, 1.0, 0.0, -7.0], np.float32)
    b = DeviceBuffer.from_host(f)
    thrust.view_mut(b).sort_by(ex, lambda l, r: (r > l) - (r < l))
    assert b.to_host_vec().view(np.uint32).tolist() == \
        np.array([2.5, 1.0, -0.0, 0.0, -7.0], np.float32).view(np.uint32).tolist()


@pytest.mark.parametrize("name,closure", [
    # sort.rs:36-49: evens first, then by value
    ("evens_first", lambda l, r: -1 if (l & 1) == 0 and (r & 1) != 0 else
     (1 if (l & 1) != 0 and (r & 1) == 0 else rust_cmp(l, r))),
    # sort.rs:100-104: parity, then value
    ("parity_then_value", lambda l, r: rust_cmp(l & 1, r & 1) or rust_cmp(l, r)),
    # sort.rs:108-112: by decade (stable)
    ("by_decade", lambda l, r: rust_cmp(l // 10, r // 10)),
])
def test_custom_comparators_rejected_before_launch(ex, name, closure):
    b = _buf(STABLE_IN)
    with pytest.raises(cub.ComparatorNotLowered):
        thrust.view_mut(b).sort_by(ex, closure)
    with pytest.raises(cub.ComparatorNotLowered):
        thrust.view_mut(b).sort_unstable_by(ex, closure)
    v = _buf(range(len(STABLE_IN)))
    with pytest.raises(cub.ComparatorNotLowered):
        thrust.view_mut(b).with_values(thrust.view_mut(v)).sort_by(ex, closure)
    assert b.to_host_vec().tolist() == STABLE_IN
    assert v.to_host_vec().tolist() == list(range(len(STABLE_IN)))


def _shuffled_unique(count):
    """comparison_sort.rs:10-20: xorshift Fisher-Yates of 0..count."""
    values = list(range(count))
    state = 0x534D4152545F534F
    m = (1 << 64) - 1
    for index in range(count - 1, 0, -1):
        state ^= (state << 13) & m
        state ^= state >> 7
        state ^= (state << 17) & m
        j = state % (index + 1)
        values[index], values[j] = values[j], values[index]
    return np.array(values, dtype=np.uint32)


def test_comparison_sort_routes(ex):
    # comparison_sort.rs:27-75
    inp = _shuffled_unique(10_003)
    assert sorted(inp.tolist()) == list(range(10_003))
    desc = list(range(10_003))[::-1]
    b = DeviceBuffer.from_host(inp)
    thrust.view_mut(b).sort_unstable_by(ex, rev_cmp)
    assert b.to_host_vec().tolist() == desc
    k, v = DeviceBuffer.from_host(inp), DeviceBuffer.from_host(inp)
    thrust.view_mut(k).with_values(thrust.view_mut(v)).sort_unstable_by(ex, rev_cmp)
    assert k.to_host_vec().tolist() == desc and v.to_host_vec().tolist() == desc
    sk = inp % np.uint32(128)
    sv = np.arange(inp.size, dtype=np.uint32)
    expected = sorted(zip(sk.tolist(), sv.tolist()), key=lambda p: p[0])
    k, v = DeviceBuffer.from_host(sk), DeviceBuffer.from_host(sv)
    thrust.view_mut(k).with_values(thrust.view_mut(v)).sort_by(ex, rust_cmp)
    assert list(zip(k.to_host_vec().tolist(), v.to_host_vec().tolist())) == expected


@pytest.mark.parametrize("n", [65_535, 65_536, 200_003])
@pytest.mark.parametrize("dt", [np.uint32, np.int64, np.float32])
def test_sort_by_stable_ties_at_lowering_sizes(ex, n, dt):
    """sort_by on both sides of the merge-sort-to-radix lowering threshold
    (integer keys) and for floats (merge sort kernels), ascending and
    descending, with index payloads: the stable order of Python's sorted()."""
    rng = np.random.default_rng(n + np.dtype(dt).itemsize)
    keys = rng.integers(-50, 50, size=n).astype(dt) if np.dtype(dt).kind != "u" else \
        rng.integers(0, 100, size=n).astype(dt)
    vals = np.arange(n, dtype=np.uint32)
    for closure, rev in ((rust_cmp, False), (rev_cmp, True)):
        k, v = DeviceBuffer.from_host(keys), DeviceBuffer.from_host(vals)
        thrust.view_mut(k).with_values(thrust.view_mut(v)).sort_by(ex, closure)
        kl = keys.tolist()
        order = sorted(range(n), key=kl.__getitem__, reverse=rev)
        assert v.to_host_vec().tolist() == order
        assert np.array_equal(k.to_host_vec(), keys[order])
