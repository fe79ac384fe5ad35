"""GPU parity tests for DeviceMerge and DeviceMergeSort through the C ABI.

Literal cases come from the reference's probe
(rccl-cub/examples/device_ordering_probe.rs:14-213); the rest compare every
output bit-for-bit with the CPU oracle (oracle/oracle.c) on the same seeded
input, across key kinds, both orders and every value width.
"""
import numpy as np
import pytest

import oracle
from rccl_amd import cub, workloads
from rccl_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu

KINDS = ["u8", "i8", "u16", "i16", "u32", "i32", "f32", "u64", "i64", "f64"]
DTYPES = {"u8": np.uint8, "i8": np.int8, "u16": np.uint16, "i16": np.int16, "u32": np.uint32,
          "i32": np.int32, "f32": np.float32, "u64": np.uint64, "i64": np.int64,
          "f64": np.float64}


def _order(descending):
    return cub.descending if descending else cub.ascending


def _random_keys(kind, n, seed, distinct=None):
    """Seeded keys of `kind`; `distinct` limits the value domain to force ties
    (centred on zero for signed and float kinds)."""
    raw = workloads.hash_range(seed, n)
    dt = np.dtype(DTYPES[kind])
    if distinct is not None:
        small = (raw % np.uint64(distinct)).astype(np.int64)
        if dt.kind != "u":
            small -= distinct // 2
        return small.astype(dt)
    if dt.kind == "f":
        # Finite floats of both signs over a wide exponent spread (no NaN).
        u = (raw >> np.uint64(11)).astype(np.float64) / float(1 << 53)
        e = (raw & np.uint64(63)).astype(np.float64) - 32.0
        return ((u - 0.5) * np.exp2(e)).astype(dt)
    top = (raw >> np.uint64(64 - 8 * dt.itemsize)).astype(np.dtype(f"u{dt.itemsize}"))
    return top.view(dt)


def _sorted(kind, keys, descending):
    s = np.sort(keys, kind="stable")
    return s[::-1].copy() if descending else s


def _values(width, n, seed):
    if width == 0:
        return None
    if width == 16:
        return workloads.hash_range(seed, 2 * n).view(np.dtype((np.void, 16)))
    dt = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[width]
    return (workloads.hash_range(seed, n) >> np.uint64(64 - 8 * width)).astype(dt)


def _dev(host):
    return DeviceBuffer.from_host(host)


def _bits(a):
    return a.view(np.dtype(f"u{a.dtype.itemsize}")) if a.dtype.kind != "V" else a.view(np.uint64)


def _merge(launch, kind, a, b, av=None, bv=None, descending=False):
    ak, bk = _dev(a), _dev(b)
    out = DeviceBuffer.empty(a.dtype, a.size + b.size)
    if av is None:
        ws = cub.device_merge_workspace(launch, a.dtype, a.size, b.size)
        cub.device_merge_keys(launch, ak, bk, ws, out, _order(descending))
        launch.synchronize()
        return out.to_host_vec()
    avd, bvd = _dev(av), _dev(bv)
    outv = DeviceBuffer.empty(av.dtype, a.size + b.size)
    ws = cub.device_merge_pairs_workspace(launch, a.dtype, av.dtype, a.size, b.size)
    cub.device_merge_pairs(launch, ak, avd, bk, bvd, ws, out, outv, _order(descending))
    launch.synchronize()
    return out.to_host_vec(), outv.to_host_vec()


def _merge_sort(launch, keys, values=None, descending=False, copy=False):
    k = _dev(keys)
    if values is None:
        ws = cub.device_merge_sort_workspace(launch, keys.dtype, keys.size)
        if copy:
            out = DeviceBuffer.empty(keys.dtype, keys.size)
            cub.device_merge_sort_keys_copy(launch, k, ws, out, _order(descending))
            launch.synchronize()
            assert np.array_equal(_bits(k.to_host_vec()), _bits(keys)), "input modified"
            return out.to_host_vec()
        cub.device_merge_sort_keys(launch, k, ws, _order(descending))
        launch.synchronize()
        return k.to_host_vec()
    v = _dev(values)
    ws = cub.device_merge_sort_pairs_workspace(launch, keys.dtype, values.dtype, keys.size)
    if copy:
        ok = DeviceBuffer.empty(keys.dtype, keys.size)
        ov = DeviceBuffer.empty(values.dtype, keys.size)
        cub.device_merge_sort_pairs_copy(launch, k, v, ws, ok, ov, _order(descending))
        launch.synchronize()
        return ok.to_host_vec(), ov.to_host_vec()
    cub.device_merge_sort_pairs(launch, k, v, ws, _order(descending))
    launch.synchronize()
    return k.to_host_vec(), v.to_host_vec()


# ---------------------------------------------------------------------------
# Literal probe cases (rccl-cub/examples/device_ordering_probe.rs).
# ---------------------------------------------------------------------------
def test_merge_keys_literal(launch):
    # :14-27
    out = _merge(launch, "i32", np.array([0, 2, 5], np.int32), np.array([0, 3, 3, 4], np.int32))
    assert out.tolist() == [0, 0, 2, 3, 3, 4, 5]


def test_merge_pairs_literal_bytes(launch):
    # :32-50: equal keys take the first range's item first.
    keys, vals = _merge(launch, "i32", np.array([0, 2, 5], np.int32),
                        np.array([0, 3, 3, 4], np.int32),
                        np.frombuffer(b"abc", np.uint8).copy(),
                        np.frombuffer(b"ABCD", np.uint8).copy())
    assert keys.tolist() == [0, 0, 2, 3, 3, 4, 5]
    assert vals.tobytes() == b"aAbBCDc"


def test_merge_pairs_i16_3623_6346(launch):
    # :52-104 (catch2 DeviceMerge::MergePairs default sizes, int16 keys, int values)
    a = (np.arange(3623) * 2).astype(np.int16)
    b = (np.arange(6346) * 2 + 1).astype(np.int16)
    av = np.arange(3623, dtype=np.int32)
    bv = (10000 + np.arange(6346)).astype(np.int32)
    keys, vals = _merge(launch, "i16", a, b, av, bv)
    ek, ev = [], []
    i = j = 0
    while i < a.size or j < b.size:
        if j == b.size or (i < a.size and a[i] <= b[j]):
            ek.append(a[i]); ev.append(av[i]); i += 1
        else:
            ek.append(b[j]); ev.append(bv[j]); j += 1
    assert keys.tolist() == [int(x) for x in ek]
    assert vals.tolist() == [int(x) for x in ev]


def test_merge_sort_literals(launch):
    # :114-121, :136-146, :167-177, :179-213
    assert _merge_sort(launch, np.array([5, 1, 3, 1, 4, 2, 0], np.int32)).tolist() == \
        [0, 1, 1, 2, 3, 4, 5]
    src = np.array([4, 1, 3, 0, 2], np.int32)
    assert _merge_sort(launch, src, copy=True).tolist() == [0, 1, 2, 3, 4]
    k, v = _merge_sort(launch, np.array([5, 1, 3, 1, 4, 2, 0], np.int32),
                       np.arange(7, dtype=np.uint32))
    assert k.tolist() == [0, 1, 1, 2, 3, 4, 5]
    assert v.tolist() == [6, 1, 3, 5, 2, 4, 0]
    k, v = _merge_sort(launch, src, np.array([40, 10, 30, 0, 20], np.uint32), copy=True)
    assert k.tolist() == [0, 1, 2, 3, 4]
    assert v.tolist() == [0, 10, 20, 30, 40]


def test_merge_sort_stability_literal(launch):
    # :124-133: sorting by key / 10 keeps equal-decade keys in input order.
    # The closure `(l / 10).cmp(r / 10)` has no prebuilt kernel; the same
    # stability is observed by sorting the decade with the key as payload.
    src = np.array([25, 14, 35, 16, 26, 34, 36, 24, 15], np.int32)
    k, v = _merge_sort(launch, src // 10, src)
    assert v.tolist() == [14, 16, 15, 25, 26, 24, 35, 34, 36]


# ---------------------------------------------------------------------------
# Oracle parity across kinds, orders and value widths.
# ---------------------------------------------------------------------------
MERGE_SHAPES = [(0, 0), (0, 5), (7, 0), (1, 1), (4095, 1), (4096, 4096), (3000, 9000),
                (50_000, 70_001)]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("descending", [False, True])
def test_merge_keys_vs_oracle(launch, kind, descending):
    for idx, (na, nb) in enumerate(MERGE_SHAPES):
        distinct = 37 if idx % 2 else None
        a = _sorted(kind, _random_keys(kind, na, 100 + idx, distinct), descending)
        b = _sorted(kind, _random_keys(kind, nb, 200 + idx, distinct), descending)
        got = _merge(launch, kind, a, b, descending=descending)
        want = oracle.merge(kind, a, b, descending=descending)
        assert np.array_equal(_bits(got), _bits(want)), (kind, na, nb)


@pytest.mark.parametrize("kind", ["u8", "i16", "u32", "f32", "u64", "f64"])
@pytest.mark.parametrize("width", [1, 2, 4, 8, 16])
def test_merge_pairs_vs_oracle(launch, kind, width):
    for idx, (na, nb) in enumerate([(1, 0), (5000, 3000), (40_000, 40_000)]):
        for descending in (False, True):
            a = _sorted(kind, _random_keys(kind, na, 300 + idx, 29), descending)
            b = _sorted(kind, _random_keys(kind, nb, 400 + idx, 29), descending)
            av, bv = _values(width, na, 500 + idx), _values(width, nb, 600 + idx)
            gk, gv = _merge(launch, kind, a, b, av, bv, descending)
            wk, wv = oracle.merge(kind, a, b, av, bv, descending)
            assert np.array_equal(_bits(gk), _bits(wk)), (kind, width, na, nb, descending)
            assert gv.tobytes() == wv.tobytes(), (kind, width, na, nb, descending)


def _sampled_shapes(kind):
    """Merges of at least 512 tiles (the sampled partition: every 2,048th A
    item bracketed against the sampled B items), with the shapes that stress
    its bounds: heavy duplicates, one side far shorter, all keys equal,
    disjoint ranges either way round, lengths that are not multiples of the
    sample stride."""
    n = 1 << 21
    dt = np.dtype(DTYPES[kind])
    rnd = lambda size, seed, distinct=None: _random_keys(kind, size, seed, distinct)
    lo, hi = (np.iinfo(dt).min, np.iinfo(dt).max)
    yield "dups", rnd(n + 3, 11, 37), rnd(n - 5, 12, 37)
    yield "uniform", rnd(n, 13), rnd(n + 2047, 14)
    yield "short_b", rnd(3 * n + 1, 15, 1000), rnd(5000, 16, 1000)
    yield "short_a", rnd(777, 17), rnd(2 * n + 17, 18)
    yield "all_equal", np.full(n + 1, 7, dt), np.full(n - 1, 7, dt)
    yield "a_before_b", np.full(n, lo, dt), np.full(n + 9, hi, dt)
    yield "b_before_a", np.full(n + 9, hi, dt), np.full(n, lo, dt)


@pytest.mark.parametrize("kind", ["u8", "i16", "u32", "i32", "u64", "i64"])
@pytest.mark.parametrize("descending", [False, True])
def test_merge_sampled_partition_vs_oracle(launch, kind, descending):
    for idx, (name, a, b) in enumerate(_sampled_shapes(kind)):
        a, b = _sorted(kind, a, descending), _sorted(kind, b, descending)
        if idx % 2:
            av, bv = _values(4, a.size, 40 + idx), _values(4, b.size, 50 + idx)
            gk, gv = _merge(launch, kind, a, b, av, bv, descending)
            wk, wv = oracle.merge(kind, a, b, av, bv, descending)
            assert np.array_equal(gv, wv), (kind, name, descending)
        else:
            gk = _merge(launch, kind, a, b, descending=descending)
            wk = oracle.merge(kind, a, b, descending=descending)
        assert np.array_equal(_bits(gk), _bits(wk)), (kind, name, descending)


SORT_SIZES = [0, 1, 2, 255, 256, 4095, 4096, 4097, 12_289, 100_000]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("descending", [False, True])
def test_merge_sort_keys_vs_oracle(launch, kind, descending):
    for idx, n in enumerate(SORT_SIZES):
        keys = _random_keys(kind, n, 700 + idx, 53 if idx % 2 else None)
        want = oracle.merge_sort(kind, keys, descending=descending)
        got = _merge_sort(launch, keys, descending=descending, copy=bool(idx % 3 == 0))
        assert np.array_equal(_bits(got), _bits(want)), (kind, n)


@pytest.mark.parametrize("kind", ["i8", "u16", "i32", "f32", "i64", "f64"])
@pytest.mark.parametrize("width", [1, 4, 8, 16])
def test_merge_sort_pairs_vs_oracle(launch, kind, width):
    for idx, n in enumerate([3, 4097, 65_537]):
        for descending in (False, True):
            keys = _random_keys(kind, n, 800 + idx, 11)
            vals = _values(width, n, 900 + idx)
            wk, wv = oracle.merge_sort(kind, keys, vals, descending)
            gk, gv = _merge_sort(launch, keys, vals, descending, copy=bool(idx % 2))
            assert np.array_equal(_bits(gk), _bits(wk)), (kind, width, n, descending)
            assert gv.tobytes() == wv.tobytes(), (kind, width, n, descending)


def test_merge_c4_scaled(launch):
    """C4 merge shape (sorted u32 in [0, 2^24), u32 payloads marking the
    source) at 2^20 per side, bit-exact with the oracle."""
    a, pa, b, pb = workloads.c4_merge_inputs(1 << 20)
    gk, gv = _merge(launch, "u32", a, b, pa, pb)
    wk, wv = oracle.merge("u32", a, b, pa, pb)
    assert np.array_equal(gk, wk)
    assert np.array_equal(gv, wv)


def test_merge_sort_c4_scaled(launch):
    """C4 merge-sort keys at 2^21, bit-exact with the oracle."""
    keys = workloads.c4_merge_sort_keys(1 << 21)
    got = _merge_sort(launch, keys)
    assert np.array_equal(got, oracle.merge_sort("u32", keys))


@pytest.mark.parametrize("kind", ["u32", "i32", "u64", "i64"])
def test_merge_sort_radix_lowering(launch, radix_ranking, kind):
    """From 65,536 items, integer keys sort through the stable radix lowering.
    Sizes on both sides of that threshold, ties (stability, with payloads
    recording the input order), both orders, in-place and copy forms."""
    for idx, n in enumerate([65_535, 65_536, 300_007]):
        for descending in (False, True):
            keys = _random_keys(kind, n, 1000 + idx, None if idx == 1 else 97)
            want = oracle.merge_sort(kind, keys, descending=descending)
            got = _merge_sort(launch, keys, descending=descending, copy=bool(idx % 2))
            assert np.array_equal(_bits(got), _bits(want)), (kind, n, descending)
            for width in (4, 16):
                vals = _values(width, n, 1100 + idx) if width == 16 else \
                    np.arange(n, dtype=np.uint32)
                wk, wv = oracle.merge_sort(kind, keys, vals, descending)
                copy = not bool(idx % 2)
                k, v = _dev(keys), _dev(vals)
                ws = cub.device_merge_sort_pairs_workspace(launch, keys.dtype, vals.dtype, n)
                if copy:
                    ok = DeviceBuffer.empty(keys.dtype, n)
                    ov = DeviceBuffer.empty(vals.dtype, n)
                    cub.device_merge_sort_pairs_copy(launch, k, v, ws, ok, ov, _order(descending))
                else:
                    ok, ov = k, v
                    cub.device_merge_sort_pairs(launch, k, v, ws, _order(descending))
                launch.synchronize()
                assert np.array_equal(_bits(ok.to_host_vec()), _bits(wk)), (kind, n, width)
                assert ov.to_host_vec().tobytes() == wv.tobytes(), (kind, n, width)
                if copy:
                    assert np.array_equal(_bits(k.to_host_vec()), _bits(keys)), "input modified"
                    assert v.to_host_vec().tobytes() == vals.tobytes(), "input modified"


@pytest.mark.parametrize("kind", ["f32", "f64"])
def test_merge_sort_float_radix_lowering_signed_zeros(launch, radix_ranking, kind):
    """Float keys from 65,536 items also sort through the radix lowering. The
    merge sort's order is IEEE `<`, under which -0.0 and +0.0 are equal: they
    must keep their input order, as the oracle's comparison merge sort keeps
    them. A quarter of the keys are signed zeros, interleaved; the rest are
    small signed values with ties, and +-inf and denormals. Payloads record
    the input order."""
    dt = np.dtype(DTYPES[kind])
    for idx, n in enumerate([65_535, 65_536, 300_007]):
        raw = workloads.hash_range(1300 + idx, n)
        keys = ((raw % np.uint64(41)).astype(np.int64) - 20).astype(dt)
        sel = raw >> np.uint64(58)  # 0..63
        keys[sel < 8] = dt.type(0.0)
        keys[(sel >= 8) & (sel < 16)] = dt.type(-0.0)
        keys[sel == 16] = dt.type(np.inf)
        keys[sel == 17] = dt.type(-np.inf)
        keys[sel == 18] = np.finfo(dt).smallest_subnormal
        keys[sel == 19] = -np.finfo(dt).smallest_subnormal
        vals = np.arange(n, dtype=np.uint32)
        for descending in (False, True):
            wk, wv = oracle.merge_sort(kind, keys, vals, descending)
            for copy in (False, True):
                gk, gv = _merge_sort(launch, keys, vals, descending, copy=copy)
                assert np.array_equal(_bits(gk), _bits(wk)), (kind, n, descending, copy)
                assert np.array_equal(gv, wv), (kind, n, descending, copy)
            zeros = (_bits(wk) << np.uint64(1) if dt.itemsize == 8 else
                     _bits(wk) << np.uint32(1)) == 0
            assert np.signbit(wk[zeros]).any() and not np.signbit(wk[zeros]).all()
            assert np.all(np.diff(wv[zeros].astype(np.int64)) > 0)  # input order


def test_merge_sort_c4_full_size(launch, radix_ranking):
    """The benchmark's C4 merge sort (2^26 u32 keys in [0, 2^24), copy form),
    bit-exact with numpy's stable sort (keys only, so any correct sort is the
    stable one)."""
    keys = workloads.c4_merge_sort_keys(1 << 26)
    got = _merge_sort(launch, keys, copy=True)
    assert np.array_equal(got, np.sort(keys, kind="stable"))


@pytest.mark.parametrize("kind", ["u32", "i64"])
@pytest.mark.parametrize("shape", ["constant", "low_byte_constant", "top_byte_only"])
def test_merge_sort_radix_lowering_trivial_passes(launch, radix_ranking, kind, shape):
    """The radix lowering skips passes whose byte is the same in every key;
    the plan must still leave a stable result in the output, in place (even
    active-pass count) and in the copy form (the input read first): every
    key equal, the lowest byte constant, only the top byte varying."""
    n = 200_003
    dt = np.dtype(DTYPES[kind])
    bits = 8 * dt.itemsize
    raw = workloads.hash_range(77, n)
    if shape == "constant":
        keys = np.full(n, 7, dtype=dt)
    elif shape == "low_byte_constant":
        keys = ((raw >> np.uint64(72 - bits)) << np.uint64(8)).astype(dt.str.replace("i", "u")) \
            .view(dt)
    else:
        keys = ((raw >> np.uint64(56)) << np.uint64(bits - 8)).astype(dt.str.replace("i", "u")) \
            .view(dt)
    vals = np.arange(n, dtype=np.uint32)
    for descending in (False, True):
        wk, wv = oracle.merge_sort(kind, keys, vals, descending)
        for copy in (False, True):
            gk, gv = _merge_sort(launch, keys, vals, descending, copy=copy)
            assert np.array_equal(_bits(gk), _bits(wk)), (shape, descending, copy)
            assert np.array_equal(gv, wv), (shape, descending, copy)
        got = _merge_sort(launch, keys, descending=descending, copy=True)
        assert np.array_equal(_bits(got), _bits(wk)), (shape, descending)


@pytest.mark.parametrize("kind", ["u32", "u64"])
@pytest.mark.parametrize("alias", ["keys", "values"])
@pytest.mark.parametrize("shape", ["one_byte", "constant", "full"])
def test_merge_sort_radix_lowering_mixed_aliasing(launch, radix_ranking, kind, alias,
                                                  shape):
    """Above the lowering threshold, keys in place with values copied (or the
    reverse): the plan must not let one pass read and write the in-place
    stream, and must write the copied stream even when no pass is needed."""
    from rccl_amd import _abi

    n = 131_075
    dt = np.dtype(DTYPES[kind])
    raw = workloads.hash_range(4242, n)
    if shape == "one_byte":
        keys = (raw >> np.uint64(56)).astype(dt)  # an odd active-pass count (one)
    elif shape == "constant":
        keys = np.full(n, 9, dtype=dt)
    else:
        keys = (raw >> np.uint64(64 - 8 * dt.itemsize)).astype(dt)
    vals = np.arange(n, dtype=np.uint32)
    wk, wv = oracle.merge_sort(kind, keys, vals, False)
    k_in, v_in = _dev(keys), _dev(vals)
    if alias == "keys":
        k_out, v_out = k_in, DeviceBuffer.zeroed(np.uint32, n)
    else:
        k_out, v_out = DeviceBuffer.zeroed(dt, n), v_in
    ws = cub.device_merge_sort_pairs_workspace(launch, dt, np.uint32, n)
    wptr, wbytes = cub._ws_ptr(ws)
    _abi.check(_abi.load().rccl_hip_merge_sort(_abi.KEY_KINDS[kind], 4, 0, k_in.ptr, v_in.ptr,
                                               k_out.ptr, v_out.ptr, n, wptr, wbytes,
                                               launch.handle))
    launch.synchronize()
    np.testing.assert_array_equal(k_out.to_host_vec(), wk)
    np.testing.assert_array_equal(v_out.to_host_vec(), wv)


@pytest.mark.parametrize("kind", ["u32", "f32"])
@pytest.mark.parametrize("descending", [False, True])
def test_merge_keys_tile_switch_at_2pow24(launch, kind, descending):
    """Keys-only merges of 4-byte keys use 12-item tiles up to 2^24 outputs
    and 16-item tiles above: both sides of the switch, and a larger merge
    with heavy duplicates, against the oracle; the workspace (one split per
    tile) shrinks across the switch."""
    half = 1 << 23
    shapes = [("at", half, half, None), ("past", half, half + 1, None),
              ("dups", (1 << 23) + 12_345, (1 << 23) + (1 << 20), 5_000)]
    for name, na, nb, distinct in shapes:
        a = _sorted(kind, _random_keys(kind, na, 71, distinct), descending)
        b = _sorted(kind, _random_keys(kind, nb, 72, distinct), descending)
        got = _merge(launch, kind, a, b, descending=descending)
        want = oracle.merge(kind, a, b, descending=descending)
        assert np.array_equal(_bits(got), _bits(want)), (kind, name, descending)
    from rccl_amd import _abi

    at, past = (_abi.workspace_bytes("rccl_hip_merge_workspace_bytes", _abi.KEY_KINDS[kind], 0,
                                     half, nb) for nb in (half, half + 1))
    assert past < at, (at, past)
