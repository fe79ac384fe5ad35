"""GPU parity tests for DeviceRadixSort through the C ABI.

Cases follow the reference's own probes
(rccl-cub/examples/device_radix_sort_keys_probe.rs and
device_radix_sort_pairs_probe.rs); every output is compared bit-for-bit with
the CPU oracle (oracle/oracle.c) on the same input.
"""
import functools

import numpy as np
import pytest

import oracle
import radix_shapes
from rccl_amd import cub, workloads
from rccl_amd.device import DeviceBuffer

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("radix_ranking")]


def _sort_keys(launch, host, descending=False):
    keys = DeviceBuffer.from_host(host)
    ws = cub.device_radix_sort_workspace(launch, host.dtype, host.size)
    if descending:
        cub.device_radix_sort_keys_descending(launch, keys, ws)
    else:
        cub.device_radix_sort_keys(launch, keys, ws)
    launch.synchronize()
    return keys.to_host_vec()


def _sort_pairs(launch, keys_host, values_host, descending=False):
    keys = DeviceBuffer.from_host(keys_host)
    values = DeviceBuffer.from_host(values_host)
    ws = cub.device_radix_sort_pairs_workspace(launch, keys_host.dtype, values_host.dtype,
                                               keys_host.size)
    if descending:
        cub.device_radix_sort_pairs_descending(launch, keys, values, ws)
    else:
        cub.device_radix_sort_pairs(launch, keys, values, ws)
    launch.synchronize()
    return keys.to_host_vec(), values.to_host_vec()


def _kind(a):
    return {np.dtype(np.uint32): "u32", np.dtype(np.int32): "i32", np.dtype(np.float32): "f32",
            np.dtype(np.uint64): "u64", np.dtype(np.int64): "i64",
            np.dtype(np.float64): "f64"}[a.dtype]


def _bits(a):
    return a.view(np.uint32 if a.dtype.itemsize == 4 else np.uint64)


def _probe_input_u32(n):
    # device_radix_sort_keys_probe.rs:36-40
    i = np.arange(n, dtype=np.uint64)
    v = (i * np.uint64(2654435761)) & np.uint64(0xFFFFFFFF)
    r = (i & np.uint64(31))
    v = ((v << r) | (v >> ((np.uint64(32) - r) & np.uint64(31)))) & np.uint64(0xFFFFFFFF)
    v = np.where(r == 0, (i * np.uint64(2654435761)) & np.uint64(0xFFFFFFFF), v)
    return v.astype(np.uint32)


def test_empty_and_single(launch):
    assert _sort_keys(launch, np.empty(0, np.uint32)).size == 0
    np.testing.assert_array_equal(_sort_keys(launch, np.array([42], np.uint32)), [42])


@pytest.mark.parametrize("n", [2, 100, 4864, 4865, 8192, 8193, 10_003, 65_537])
@pytest.mark.parametrize("descending", [False, True])
def test_u32_sizes(launch, n, descending):
    host = _probe_input_u32(n)
    host[min(17, n - 1)] = 0
    host[min(29, n - 1)] = 0xFFFFFFFF
    got = _sort_keys(launch, host, descending)
    want = oracle.radix_sort("u32", host, descending=descending)
    np.testing.assert_array_equal(got, want)


def test_c1_u32_2pow20(launch):
    host = workloads.c1_keys()
    got = _sort_keys(launch, host)
    np.testing.assert_array_equal(got, np.sort(host))
    np.testing.assert_array_equal(got, oracle.radix_sort("u32", host))


@pytest.mark.parametrize("log2n", [20, 24])
def test_reference_benchmark_input(launch, log2n):
    """The reference benchmark's xorshift keys (benchmarks/ordering-reference.cu:23-33), at
    2^20 and at its published size 2^24, against the oracle and numpy's sort."""
    host = workloads.reference_bench_u32(1 << log2n)
    got = _sort_keys(launch, host)
    np.testing.assert_array_equal(got, np.sort(host))
    if log2n == 20:
        np.testing.assert_array_equal(got, oracle.radix_sort("u32", host))


def test_signed_descending_literal(launch):
    # device_radix_sort_keys_probe.rs:75-97
    got = _sort_keys(launch, np.array([0, -1, -2**31, 7, -9, 2**31 - 1, -1, 0], np.int32), True)
    np.testing.assert_array_equal(got, [2**31 - 1, 7, 0, 0, -1, -1, -9, -2**31])
    got = _sort_keys(launch, np.array([0, -1, -2**63, 7, -9, 2**63 - 1, -1, 0], np.int64), True)
    np.testing.assert_array_equal(got, [2**63 - 1, 7, 0, 0, -1, -1, -9, -2**63])


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_float_signed_zero_literal(launch, dt):
    # device_radix_sort_keys_probe.rs:99-119 and :175-199
    host = np.array([3.0, -0.0, -np.inf, 0.0, -7.5, np.inf], dt)
    got = _sort_keys(launch, host)
    want = np.array([-np.inf, -7.5, -0.0, 0.0, 3.0, np.inf], dt)
    np.testing.assert_array_equal(_bits(got), _bits(want))


def test_nan_bit_order_literal(launch):
    # device_radix_sort_keys_probe.rs:121-173
    nq, ns, ps, pq = 0xFFC00001, 0xFF800001, 0x7F800001, 0x7FC00001
    one, mone = 0x3F800000, 0xBF800000
    host = np.array([pq, one, ns, nq, mone, ps], np.uint32).view(np.float32)
    asc = _sort_keys(launch, host)
    np.testing.assert_array_equal(asc.view(np.uint32), [nq, ns, mone, one, ps, pq])
    desc = _sort_keys(launch, host, True)
    np.testing.assert_array_equal(desc.view(np.uint32), [pq, ps, one, mone, ns, nq])
    nq, ns, ps, pq = (0xFFF8000000000001, 0xFFF0000000000001, 0x7FF0000000000001,
                      0x7FF8000000000001)
    one, mone = 0x3FF0000000000000, 0xBFF0000000000000
    host = np.array([pq, one, ns, nq, mone, ps], np.uint64).view(np.float64)
    asc = _sort_keys(launch, host)
    np.testing.assert_array_equal(asc.view(np.uint64), [nq, ns, mone, one, ps, pq])
    desc = _sort_keys(launch, host, True)
    np.testing.assert_array_equal(desc.view(np.uint64), [pq, ps, one, mone, ns, nq])


@pytest.mark.parametrize("descending", [False, True])
def test_low_entropy_and_uniform(launch, descending):
    # device_radix_sort_keys_probe.rs:248-294
    n = (1 << 17) + 3
    i = np.arange(n, dtype=np.uint64)
    entropy = ((i * np.uint64(2654435761)) & np.uint64(31)).astype(np.uint32)
    got = _sort_keys(launch, entropy, descending)
    want = np.sort(entropy)[::-1] if descending else np.sort(entropy)
    np.testing.assert_array_equal(got, want)
    uniform = np.full(n, 4, np.uint32)
    np.testing.assert_array_equal(_sort_keys(launch, uniform, descending), uniform)


@pytest.mark.parametrize("kind", ["u32", "i32", "f32", "u64", "i64", "f64"])
@pytest.mark.parametrize("descending", [False, True])
def test_all_kinds_random_bits(launch, kind, descending):
    n = 50_001
    dt = np.dtype(oracle.KIND_DTYPES[kind])
    raw = workloads.hash_range(0xABCDEF + 7 * dt.itemsize, n)
    if dt.itemsize == 4:
        host = (raw >> np.uint64(32)).astype(np.uint32).view(dt)
    else:
        host = raw.view(dt)
    host = host.copy()
    if dt.kind == "f":
        _bits(host)[::97] = 0
        _bits(host)[1::89] = 1 << (dt.itemsize * 8 - 1)
    got = _sort_keys(launch, host, descending)
    want = oracle.radix_sort(kind, host, descending=descending)
    np.testing.assert_array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("value_dtype", [np.uint8, np.uint16, np.int32, np.uint64])
@pytest.mark.parametrize("descending", [False, True])
def test_pairs_narrow_domain(launch, value_dtype, descending):
    # device_radix_sort_pairs_probe.rs:33-99: narrow key domain, index values.
    keys = _probe_input_u32(10_003) & np.uint32(0x3FF)
    values = np.arange(keys.size).astype(value_dtype)
    gk, gv = _sort_pairs(launch, keys, values, descending)
    wk, wv = oracle.radix_sort("u32", keys, values, descending=descending)
    np.testing.assert_array_equal(gk, wk)
    np.testing.assert_array_equal(gv, wv)


@pytest.mark.parametrize("kind", ["u32", "i64"])
@pytest.mark.parametrize("width", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("descending", [False, True])
def test_pairs_every_value_width_multi_tile(launch, kind, width, descending):
    """Every value width through the onesweep passes (100,003 items: several
    tiles, a partial last one), including 16-byte values, whose payload
    bytes are random so a mixed-up word would show. Keys are 10 bits wide
    (ties in every tile); outputs are bit-exact with the oracle."""
    dt = np.dtype(oracle.KIND_DTYPES[kind])
    n = 100_003
    raw = workloads.hash_range(4242 + width, n)
    keys = (raw >> np.uint64(54)).astype(np.dtype(f"u{dt.itemsize}")).view(dt)
    if width == 16:
        vals = workloads.hash_range(77, 2 * n).view(np.dtype((np.void, 16)))
    else:
        vals = np.arange(n).astype({1: np.uint8, 2: np.uint16, 4: np.uint32,
                                    8: np.uint64}[width])
    gk, gv = _sort_pairs(launch, keys, vals, descending)
    wk, wv = oracle.radix_sort(kind, keys, vals, descending=descending)
    assert np.array_equal(_bits(gk), _bits(wk))
    assert np.array_equal(gv.view(np.uint8), wv.view(np.uint8))


def test_pairs_u64_keys_u32_values(launch):
    keys, values = workloads.c2_uniform(1 << 18)
    gk, gv = _sort_pairs(launch, keys, values)
    wk, wv = oracle.radix_sort("u64", keys, values)
    np.testing.assert_array_equal(gk, wk)
    np.testing.assert_array_equal(gv, wv)


def test_pairs_float_literal(launch):
    # device_radix_sort_pairs_probe.rs:177-214
    keys = np.array([1.25, -0.0, np.inf, -3.5, 0.0, -np.inf], np.float32)
    values = np.array([4, 2, 5, 1, 3, 0], np.int32)
    gk, gv = _sort_pairs(launch, keys, values)
    want = np.array([-np.inf, -3.5, -0.0, 0.0, 1.25, np.inf], np.float32)
    np.testing.assert_array_equal(gk.view(np.uint32), want.view(np.uint32))
    np.testing.assert_array_equal(gv, [0, 1, 2, 3, 4, 5])


@pytest.mark.parametrize("descending", [False, True])
def test_window_double_buffer(launch, descending):
    # device_radix_sort_keys_probe.rs:296-339: bits 0..24 (three passes).
    i = np.arange(10_003, dtype=np.uint64)
    low = (i * np.uint64(2654435761)) & np.uint64(0x00FFFFFF)
    host = (((i & np.uint64(0xFF)) << np.uint64(24)) | low).astype(np.uint32)
    first = DeviceBuffer.from_host(host)
    second = DeviceBuffer.zeroed(np.uint32, host.size)
    buffers = cub.DoubleBuffer.new(first, second)
    ws = cub.device_radix_sort_keys_buffer_workspace(launch, np.uint32, host.size)
    if descending:
        cub.device_radix_sort_keys_buffer_descending(launch, buffers, range(0, 24), ws)
    else:
        cub.device_radix_sort_keys_buffer(launch, buffers, range(0, 24), ws)
    launch.synchronize()
    got = buffers.current().to_host_vec()
    field = host & np.uint32(0x00FFFFFF)
    order = np.argsort(field.astype(np.int64) * (-1 if descending else 1), kind="stable")
    np.testing.assert_array_equal(got, host[order])
    np.testing.assert_array_equal(got, oracle.radix_sort("u32", host, descending=descending,
                                                         begin_bit=0, end_bit=24))


def test_window_noop_and_invalid(launch):
    # device_radix_sort_keys_probe.rs:341-391
    host = np.array([9, 1, 7, 3], np.uint32)
    first = DeviceBuffer.from_host(host)
    second = DeviceBuffer.from_host(np.array([99, 99, 99, 99], np.uint32))
    buffers = cub.DoubleBuffer.new(first, second)
    ws = cub.device_radix_sort_keys_buffer_workspace(launch, np.uint32, 4)
    cub.device_radix_sort_keys_buffer(launch, buffers, range(12, 12), ws)
    assert buffers.current_is_first()
    np.testing.assert_array_equal(buffers.current().to_host_vec(), host)
    with pytest.raises(cub.DeviceAlgorithmError) as err:
        cub.device_radix_sort_keys_buffer(launch, buffers, range(25, 17), ws)
    assert err.value.kind == "InvalidBitRange"
    assert (err.value.begin, err.value.end, err.value.key_bits) == (25, 17, 32)
    np.testing.assert_array_equal(buffers.current().to_host_vec(), host)
    cub.device_radix_sort_keys_buffer(launch, buffers, range(0, 8), ws)
    launch.synchronize()
    np.testing.assert_array_equal(buffers.current().to_host_vec(), [1, 3, 7, 9])


@pytest.mark.parametrize("dtype,vdtype,n,window,flipped", [
    (np.uint32, None, 100, (0, 32), True),
    (np.uint32, None, 4864, (0, 32), True),
    (np.uint32, None, 4865, (0, 32), False),
    (np.uint32, None, 100, (0, 24), True),
    (np.uint64, None, 2304, (0, 64), True),
    (np.uint64, None, 2305, (0, 64), False),
    (np.uint32, np.uint64, 2304, (0, 32), True),
    (np.uint32, np.uint64, 2305, (0, 32), False),
    (np.int32, np.uint32, 4864, (0, 16), True),
])
def test_double_buffer_selector_parity(launch, dtype, vdtype, n, window, flipped):
    """The selector ends where the reference leaves it: its single-tile route
    (n <= 256 * 19 * 4 / max(item bytes, 4), rccl-cub/src/workspace.rs:22-66)
    flips once, the onesweep route once per 8-bit pass
    (rccl-cub/src/radix.rs:470-548)."""
    raw = (np.arange(n, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15)) >> np.uint64(17)
    host = raw.astype(np.dtype(dtype).str.replace("i", "u")).view(dtype)
    kind = _kind(host)
    k0, k1 = DeviceBuffer.from_host(host), DeviceBuffer.zeroed(dtype, n)
    if vdtype is None:
        buffers = cub.DoubleBuffer.new(k0, k1)
        ws = cub.device_radix_sort_keys_buffer_workspace(launch, dtype, n)
        cub.device_radix_sort_keys_buffer(launch, buffers, range(*window), ws)
        launch.synchronize()
        got = buffers.current().to_host_vec()
        want = oracle.radix_sort(kind, host, begin_bit=window[0], end_bit=window[1])
    else:
        vals = np.arange(n, dtype=vdtype)
        v0, v1 = DeviceBuffer.from_host(vals), DeviceBuffer.zeroed(vdtype, n)
        buffers = cub.DoubleBuffer.paired((k0, v0), (k1, v1))
        ws = cub.device_radix_sort_pairs_buffer_workspace(launch, dtype, vdtype, n)
        cub.device_radix_sort_pairs_buffer(launch, buffers, range(*window), ws)
        launch.synchronize()
        ck, cv = buffers.current()
        got = ck.to_host_vec()
        want, want_v = oracle.radix_sort(kind, host, vals, begin_bit=window[0],
                                         end_bit=window[1])
        np.testing.assert_array_equal(cv.to_host_vec(), want_v)
    np.testing.assert_array_equal(_bits(got), _bits(want))
    assert buffers.current_is_first() == (not flipped)


def _single_tile_items(key_bytes, value_bytes):
    # The reference's single-tile capacity (rccl-cub/src/workspace.rs:22-66).
    return 256 * max(1, 19 * 4 // max(key_bytes, value_bytes, 4))


def _value_array(width, n):
    if width == 16:
        return workloads.hash_range(99, 2 * n).view(np.dtype((np.void, 16)))
    dt = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[width]
    return (np.arange(n, dtype=np.uint64) % np.uint64(1 << (8 * width - 1))).astype(dt)


@pytest.mark.parametrize("kind,width", [("u32", 0), ("i32", 4), ("f32", 8), ("u64", 0),
                                        ("i64", 4), ("f64", 1), ("u32", 16), ("u64", 2),
                                        ("f32", 0), ("u64", 8)])
@pytest.mark.parametrize("descending", [False, True])
def test_single_tile_route(launch, kind, width, descending):
    """Inputs up to the single-tile capacity sort in one launch (one block,
    every pass in LDS), bit-exact with the oracle, ties in input order."""
    from rccl_amd import _abi

    dt = np.dtype(oracle.KIND_DTYPES[kind])
    limit = _single_tile_items(dt.itemsize, width)
    for n in (1, 2, 63, 64, 65, 257, limit - 1, limit):
        raw = workloads.hash_range(17 * n + width, n)
        bits = (raw >> np.uint64(64 - 8 * dt.itemsize)).astype(np.dtype(f"u{dt.itemsize}"))
        bits[::5] = bits[0]  # ties
        if dt.kind == "f":
            bits[1::7] = 0
            bits[2::11] = 1 << (8 * dt.itemsize - 1)
        host = bits.view(dt)
        keys = DeviceBuffer.from_host(host)
        if width:
            vals_h = _value_array(width, n)
            vals = DeviceBuffer.from_host(vals_h)
            ws = cub.device_radix_sort_pairs_workspace(launch, dt, vals_h.dtype, n)
        else:
            ws = cub.device_radix_sort_workspace(launch, dt, n)
        _abi.timing_read()
        _abi.timing_enable(True)
        try:
            if width:
                (cub.device_radix_sort_pairs_descending if descending
                 else cub.device_radix_sort_pairs)(launch, keys, vals, ws)
            else:
                (cub.device_radix_sort_keys_descending if descending
                 else cub.device_radix_sort_keys)(launch, keys, ws)
            launch.synchronize()
        finally:
            launches = [name for name, _ms, _items in _abi.timing_read()]
            _abi.timing_enable(False)
        assert launches == ["radix_single_tile"], (n, launches)
        if width:
            wk, wv = oracle.radix_sort(kind, host, vals_h, descending=descending)
            assert np.array_equal(vals.to_host_vec().view(np.uint8), wv.view(np.uint8)), n
        else:
            wk = oracle.radix_sort(kind, host, descending=descending)
        assert np.array_equal(_bits(keys.to_host_vec()), _bits(wk)), n


@pytest.mark.parametrize("window", [(0, 24), (8, 9), (3, 32), (0, 16)])
def test_single_tile_windows_flip_once(launch, window):
    """The DoubleBuffer form of a single-tile sort leaves the result in the
    other buffer whatever the number of passes (one flip, as the
    reference's single-tile route)."""
    n = 4_000
    host = workloads.uniform_u32(n, 31 + window[0])
    vals = np.arange(n, dtype=np.uint32)
    k0, k1 = DeviceBuffer.from_host(host), DeviceBuffer.zeroed(np.uint32, n)
    v0, v1 = DeviceBuffer.from_host(vals), DeviceBuffer.zeroed(np.uint32, n)
    buffers = cub.DoubleBuffer.paired((k0, v0), (k1, v1))
    ws = cub.device_radix_sort_pairs_buffer_workspace(launch, np.uint32, np.uint32, n)
    cub.device_radix_sort_pairs_buffer(launch, buffers, range(*window), ws)
    launch.synchronize()
    assert not buffers.current_is_first()
    wk, wv = oracle.radix_sort("u32", host, vals, begin_bit=window[0], end_bit=window[1])
    ck, cv = buffers.current()
    np.testing.assert_array_equal(ck.to_host_vec(), wk)
    np.testing.assert_array_equal(cv.to_host_vec(), wv)
    np.testing.assert_array_equal(k0.to_host_vec(), host)  # the input is left as it was


# Both tile shapes: plain sorts of at most 512 small tiles use 256-thread
# blocks with half the items; one item more takes the large tiles. Inputs and
# oracle outputs are shared by the ranking modes.
@functools.lru_cache(maxsize=4)
def _threshold_case(kind, width, n, descending):
    dt = np.dtype(oracle.KIND_DTYPES[kind])
    raw = workloads.hash_range(0x51A11 + 131 * dt.itemsize + width, n)
    keys = ((raw >> np.uint64(32)).astype(np.uint32) if dt.itemsize == 4 else raw).view(dt)
    keys = keys.copy()
    if dt.kind == "f":
        _bits(keys)[::97] = 0
        _bits(keys)[1::89] = 1 << (dt.itemsize * 8 - 1)
    if width == 0:
        return keys, None, oracle.radix_sort(kind, keys, descending=descending), None
    if width == 16:
        values = workloads.hash_range(0xBEEF, 2 * n).view(np.dtype("V16"))
    else:
        values = np.arange(n, dtype=np.uint64).astype(np.dtype(f"u{width}"))
    wk, wv = oracle.radix_sort(kind, keys, values, descending=descending)
    return keys, values, wk, wv


@pytest.mark.parametrize("side", ["small_max", "large_min"])
@pytest.mark.parametrize("kind,width", [(k, 0) for k in ("u32", "i32", "f32", "u64", "i64", "f64")]
                         + [("u32", w) for w in (1, 2, 4, 8, 16)] + [("u64", 4), ("u64", 16)])
@pytest.mark.parametrize("descending", [False, True])
def test_tile_shape_threshold(launch, kind, width, side, descending):
    dt = np.dtype(oracle.KIND_DTYPES[kind])
    n = radix_shapes.small_tile_max(dt.itemsize, width) + (side == "large_min")
    keys, values, wk, wv = _threshold_case(kind, width, n, descending)
    if values is None:
        got = _sort_keys(launch, keys, descending)
        np.testing.assert_array_equal(_bits(got), _bits(wk))
    else:
        gk, gv = _sort_pairs(launch, keys, values, descending)
        np.testing.assert_array_equal(_bits(gk), _bits(wk))
        assert np.array_equal(gv, wv)


@pytest.mark.parametrize("tiles", [1, 2, 15, 16, 17, 64, 241, 511])
@pytest.mark.parametrize("delta", [-1, 0, 1])
def test_small_tile_counts(launch, tiles, delta):
    """Plain sorts whose small-tile count lands on, just below and just past
    multiples of the tile (look-back groups of 16, XCD runs of 8): keys and
    u64 + u32 pairs against the oracle."""
    for kb, vb, kind in ((4, 0, "u32"), (8, 4, "u64")):
        tile = radix_shapes.SMALL_THREADS * max(1, radix_shapes.items(kb, vb) // 2)
        n = tiles * tile + delta
        if n < 1 or n > radix_shapes.small_tile_max(kb, vb):
            continue
        raw = workloads.hash_range(0x7A11 + tiles * 7 + delta, n)
        if vb == 0:
            keys = (raw >> np.uint64(40)).astype(np.uint32)  # 24-bit keys: ties
            np.testing.assert_array_equal(_sort_keys(launch, keys),
                                          oracle.radix_sort(kind, keys))
        else:
            keys = raw >> np.uint64(20)
            values = np.arange(n, dtype=np.uint32)
            gk, gv = _sort_pairs(launch, keys, values)
            wk, wv = oracle.radix_sort(kind, keys, values)
            np.testing.assert_array_equal(gk, wk)
            np.testing.assert_array_equal(gv, wv)


def _skewed_bits(n, nbytes, nhot, seed, runs):
    """Random keys of `nbytes` bytes where each of `nhot` dictionary values
    takes about 11% of the positions, so that every byte has up to `nhot`
    digits above 1/16 of the keys (the onesweep's hot digits; more than four
    leaves the rest on the counting atomics). With `runs`, blocks of 3,000
    keys are sorted, so that whole 64-key items share a hot or a cold digit."""
    raw = workloads.hash_range(seed, n)
    pick = workloads.hash_range(seed ^ 0x5EED, n)
    dictionary = workloads.hash_range(seed ^ 0xD1C7, max(nhot, 1))
    slot = (pick >> np.uint64(40)) % np.uint64(9)  # slots 0..nhot-1 hot
    hot = slot < np.uint64(nhot)
    bits = np.where(hot, dictionary[np.minimum(slot, np.uint64(max(nhot, 1) - 1)).astype(np.int64)],
                    raw)
    if nbytes == 4:
        bits = (bits >> np.uint64(32)).astype(np.uint32)
    if runs:
        for s in range(0, n, 3000):
            bits[s:s + 3000].sort()
    return bits


@pytest.mark.parametrize("nhot", [1, 2, 4, 6])
@pytest.mark.parametrize("runs", [False, True])
@pytest.mark.parametrize("kind", ["u32", "f32", "u64"])
@pytest.mark.parametrize("descending", [False, True])
def test_skewed_digits(launch, nhot, runs, kind, descending):
    """Passes with up to four hot digits count and rank those digits by
    ballot instead of LDS atomics; ragged sizes put dummies in the last
    tile."""
    dt = np.dtype(oracle.KIND_DTYPES[kind])
    n = 1_000_003 if nhot % 2 else 3 * 17_408 + 1_234
    host = _skewed_bits(n, dt.itemsize, nhot, 0x5CE3 + nhot, runs).view(dt)
    got = _sort_keys(launch, host, descending)
    want = oracle.radix_sort(kind, host, descending=descending)
    np.testing.assert_array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("nhot", [1, 3, 5])
@pytest.mark.parametrize("descending", [False, True])
def test_skewed_digits_pairs_stable(launch, nhot, descending):
    """u64 keys with u32 index values (the C2 pair shape): ties among the
    hot keys must keep their input order."""
    n = 700_001
    keys = _skewed_bits(n, 8, nhot, 0xA11 + nhot, False)
    vals = np.arange(n, dtype=np.uint32)
    got_k, got_v = _sort_pairs(launch, keys, vals, descending)
    want_k, want_v = oracle.radix_sort("u64", keys, vals, descending=descending)
    np.testing.assert_array_equal(got_k, want_k)
    np.testing.assert_array_equal(got_v, want_v)


@pytest.mark.parametrize("kind", ["u32", "f32", "u64"])
@pytest.mark.parametrize("descending", [False, True])
def test_locally_skewed_stretch(launch, kind, descending):
    """A pass that is not skewed as a whole (no digit holds 1/16 of the keys)
    but has a skewed stretch: 5% of the input, contiguous, is 80% one value.
    Waves in that stretch take the skewed ranking on their own, others the
    uniform one, in the same blocks."""
    dt = np.dtype(oracle.KIND_DTYPES[kind])
    n = 1_000_003
    bits = workloads.hash_range(0x10CA1, n)
    lo, hi = 300_001, 300_001 + n // 20
    pick = workloads.hash_range(0x10CA2, hi - lo) % np.uint64(5)
    bits[lo:hi] = np.where(pick < np.uint64(4), bits[lo], bits[lo:hi])
    if dt.itemsize == 4:
        bits = (bits >> np.uint64(32)).astype(np.uint32)
    host = bits.view(dt)
    got = _sort_keys(launch, host, descending)
    want = oracle.radix_sort(kind, host, descending=descending)
    np.testing.assert_array_equal(_bits(got), _bits(want))
    if kind == "u64":
        vals = np.arange(n, dtype=np.uint32)
        gk, gv = _sort_pairs(launch, host, vals, descending)
        wk, wv = oracle.radix_sort("u64", host, vals, descending=descending)
        np.testing.assert_array_equal(gk, wk)
        np.testing.assert_array_equal(gv, wv)


@pytest.mark.parametrize("n", [1_000_003, 3 * 17_408 + 1, 65_537])
def test_u64_keys_off_16_byte_boundary(launch, n):
    """8-byte keys whose buffer starts 8 bytes past a 16-byte boundary (the
    histogram loads two keys per lane from the first 16-byte boundary on and
    counts the key before it separately), keys-only and pairs."""
    import torch

    host = workloads.hash_range(0x0FF5E7, n + 1)
    big = torch.from_numpy(host.view(np.int64)).to("cuda")
    view = big[1:]  # 8 bytes past the allocation's start
    assert view.data_ptr() % 16 == 8
    keys = DeviceBuffer(view, np.uint64, n)
    ws = cub.device_radix_sort_workspace(launch, np.uint64, n)
    cub.device_radix_sort_keys(launch, keys, ws)
    launch.synchronize()
    np.testing.assert_array_equal(keys.to_host_vec(), oracle.radix_sort("u64", host[1:]))
    big.copy_(torch.from_numpy(host.view(np.int64)))
    vals = DeviceBuffer.from_host(np.arange(n, dtype=np.uint32))
    keys = DeviceBuffer(big[1:], np.uint64, n)
    ws = cub.device_radix_sort_pairs_workspace(launch, np.uint64, np.uint32, n)
    cub.device_radix_sort_pairs(launch, keys, vals, ws)
    launch.synchronize()
    wk, wv = oracle.radix_sort("u64", host[1:], np.arange(n, dtype=np.uint32))
    np.testing.assert_array_equal(keys.to_host_vec(), wk)
    np.testing.assert_array_equal(vals.to_host_vec(), wv)
