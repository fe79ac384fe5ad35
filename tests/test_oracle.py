"""CPU checks that pin the oracle (oracle/oracle.c) before it is trusted.

Each oracle function is checked against
  * the literal vectors of the reference's own probes and tests
    (tests/golden/reference_vectors.json, each case citing its source), and
  * an independent restatement that shares no code with the oracle: numpy's
    stable argsort over the order-preserving key transform for radix sort,
    `heapq.merge` for merge, Python's stable `sorted` for merge sort, and
    multiset (Counter) algebra plus a per-run value rule for the set
    operations,
chosen so that a plausible mistake (a tie broken the wrong way, a missing
sign flip, a wrong ±0 rule, values taken from the wrong range) fails.
"""
import collections
import heapq
import json
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.json")
NP = {"u8": np.uint8, "i8": np.int8, "u16": np.uint16, "i16": np.int16, "u32": np.uint32,
      "i32": np.int32, "f32": np.float32, "u64": np.uint64, "i64": np.int64, "f64": np.float64}
BITS_OF = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}
OPS = ["union", "intersection", "difference", "symmetric_difference"]


def _keys(case, field, kind):
    vals = case[field]
    if case.get("float_bits"):
        bits = np.array([int(v, 16) for v in vals], dtype=BITS_OF[np.dtype(NP[kind]).itemsize])
        return bits.view(NP[kind])
    return np.array(vals, dtype=NP[kind])


def _bits(a):
    a = np.asarray(a)
    return a.view(BITS_OF[a.dtype.itemsize])


def _golden_cases():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _golden_cases(), ids=lambda c: c["id"])
def test_oracle_reproduces_reference_vectors(case):
    if case["op"] == "record_sort":
        rows = np.array(case["rows"], dtype=np.uint32)
        pay = None if "payloads" not in case else np.array(case["payloads"],
                                                          dtype=NP[case["payload_dtype"]])
        out_rows, out_pay = oracle.record_sort(rows, pay)
        assert out_rows.tolist() == case["expected_rows"]
        if "expected_payloads" in case:
            assert out_pay.tolist() == case["expected_payloads"]
        return
    if case["op"] in ("unique", "reduce_by_key"):
        _check_group_case(case)
        return
    kind, desc = case["kind"], case["descending"]
    vdt = NP.get(case.get("value_dtype", ""), None)
    if case["op"] == "radix_sort":
        keys = _keys(case, "keys", kind)
        vals = None if "values" not in case else np.array(case["values"], dtype=vdt)
        out = oracle.radix_sort(kind, keys, vals, desc, case.get("begin_bit", 0),
                                case.get("end_bit"))
    elif case["op"] == "merge":
        a, b = _keys(case, "a", kind), _keys(case, "b", kind)
        if "a_values" in case:
            out = oracle.merge(kind, a, b, np.array(case["a_values"], vdt),
                               np.array(case["b_values"], vdt), desc)
        else:
            out = oracle.merge(kind, a, b, descending=desc)
    elif case["op"] == "merge_sort":
        keys = _keys(case, "keys", kind)
        vals = None if "values" not in case else np.array(case["values"], dtype=vdt)
        out = oracle.merge_sort(kind, keys, vals, desc)
    else:
        if "a_range" in case:  # arithmetic ranges: materialised here for the oracle
            a, b = _arith(case["a_range"], kind), _arith(case["b_range"], kind)
        else:
            a, b = _keys(case, "a", kind), _keys(case, "b", kind)
        av = None if "a_values" not in case else np.array(case["a_values"], vdt)
        bv = None if "b_values" not in case else np.array(case["b_values"], vdt)
        out = oracle.set_op(case["set_op"], kind, a, b, av, bv, desc)
        assert oracle.set_op(case["set_op"], kind, a, b, descending=desc,
                             count_only=True) == len(case["expected_keys"])
    keys_out, vals_out = (out if isinstance(out, tuple) else (out, None))
    assert np.array_equal(_bits(keys_out), _bits(_keys(case, "expected_keys", kind)))
    if "expected_values" in case:
        assert vals_out.tolist() == case["expected_values"]


def _group_case_arrays(case):
    """Keys, payloads, values and expected outputs of a unique/reduce golden case."""
    keys = np.array(case["keys"], dtype=NP[case["kind"]])
    pays = None
    if "payloads" in case:
        pays = np.array(case["payloads"], dtype=NP[case["payload_dtype"]])
    vals = None
    if "values" in case:
        vals = np.array(case["values"], dtype=oracle.GROUP_VALUE_DTYPES[case["group_op"]])
    elif "values_f64_bits" in case:
        vals = np.array(case["values_f64_bits"], dtype=np.uint64).view(np.float64)
    if "expected_values_f64_bits" in case:
        exp_vals = np.array(case["expected_values_f64_bits"], dtype=np.uint64)
    elif "expected_values" in case:
        exp_vals = np.array(case["expected_values"], dtype=np.uint64)
    else:
        exp_vals = None
    return keys, pays, vals, exp_vals


def _run_lengths_first(keys):
    """Indices of run heads (first of each run of equal adjacent keys)."""
    return [i for i in range(len(keys)) if i == 0 or keys[i - 1] != keys[i]]


def _check_group_case(case):
    keys, pays, vals, exp_vals = _group_case_arrays(case)
    heads = _run_lengths_first(keys)
    if case["op"] == "unique":
        out = oracle.unique(keys, case["kind"])
        assert out.tolist() == case["expected_keys"]
        # The payload of a run is its first item's.
        assert pays[heads].tolist() == case["expected_payloads"]
        return
    out_k, out_v = oracle.reduce_by_key(keys, vals, case["group_op"], case["kind"])
    assert out_k.tolist() == case["expected_keys"]
    assert np.array_equal(out_v.view(np.uint64) if out_v.dtype == np.float64 else
                          out_v.astype(np.uint64), exp_vals)
    if pays is not None:
        assert pays[heads].tolist() == case["expected_payloads"]


def _arith(desc, kind):
    """Items start + step * i of an arithmetic range, wrapping in the kind's width."""
    start, step, n = desc
    dt = np.dtype(NP[kind])
    u = np.dtype(f"u{dt.itemsize}")
    wrap = 1 << (8 * dt.itemsize)
    vals = [(start + step * i) % wrap for i in range(n)]
    return np.array(vals, dtype=np.uint64).astype(u).view(dt)


# ---------------------------------------------------------------------------
# Radix sort vs an independent numpy restatement of the key transform
# (rccl-cub/src/ordering_backend/radix.rs:75-337): unsigned identity, signed
# sign flip, float `neg ? !raw : raw ^ sign`, descending = complement, and for
# float digits the ordered pattern 0x7f..f is read as 0x80..0 so that +0 and
# -0 tie.
# ---------------------------------------------------------------------------
def _np_ordered(kind, raw_bits, descending):
    width = raw_bits.dtype.itemsize * 8
    ut = raw_bits.dtype.type
    sign = ut(1 << (width - 1))
    if kind[0] == "u":
        o = raw_bits.copy()
    elif kind[0] == "i":
        o = raw_bits ^ sign
    else:
        neg = (raw_bits & sign) != 0
        o = np.where(neg, ~raw_bits, raw_bits ^ sign).astype(raw_bits.dtype)
    if descending:
        o = ~o
    if kind[0] == "f":
        o = np.where(o == ut((1 << (width - 1)) - 1), sign, o).astype(raw_bits.dtype)
    return o


def _np_radix(kind, keys, values, descending, begin, end):
    bits = _bits(keys)
    width = bits.dtype.itemsize * 8
    end = width if end is None else end
    src = _np_ordered(kind, bits, descending).astype(np.uint64)
    mask = np.uint64((1 << (end - begin)) - 1) if end - begin < 64 else np.uint64(~0 & (2**64 - 1))
    digit = (src >> np.uint64(begin)) & mask
    order = np.argsort(digit, kind="stable")
    return keys[order], (None if values is None else values[order])


def _special_float_keys(kind, n, seed):
    rng = np.random.default_rng(seed)
    dt = np.dtype(NP[kind])
    ut = BITS_OF[dt.itemsize]
    raw = rng.integers(0, np.iinfo(ut).max, size=n, dtype=ut, endpoint=True)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -np.nan, 1.0, -1.0,
                         np.finfo(dt).tiny, -np.finfo(dt).tiny, np.finfo(dt).max,
                         np.finfo(dt).smallest_subnormal], dtype=dt).view(ut)
    pos = rng.integers(0, n, size=n // 3)
    raw[pos] = specials[rng.integers(0, specials.size, size=pos.size)]
    return raw.view(dt)


@pytest.mark.parametrize("kind", ["u32", "i32", "f32", "u64", "i64", "f64"])
@pytest.mark.parametrize("descending", [False, True])
def test_radix_oracle_vs_numpy(kind, descending):
    n = 20_000
    dt = np.dtype(NP[kind])
    width = dt.itemsize * 8
    rng = np.random.default_rng(7 + width)
    if dt.kind == "f":
        keys = _special_float_keys(kind, n, 11 + width)
    else:
        ut = BITS_OF[dt.itemsize]
        keys = rng.integers(0, np.iinfo(ut).max, size=n, dtype=ut, endpoint=True).view(dt)
        keys[rng.integers(0, n, size=n // 4)] = keys[5]  # heavy ties
        keys[:4] = np.array([np.iinfo(dt).min, np.iinfo(dt).max, 0, 1], dtype=dt)
    values = np.arange(n, dtype=np.uint32)
    for begin, end in [(0, None), (0, width // 2), (3, width - 5), (width - 8, width), (5, 5)]:
        got_k, got_v = oracle.radix_sort(kind, keys, values, descending, begin, end)
        want_k, want_v = _np_radix(kind, keys, values, descending, begin, end)
        assert np.array_equal(_bits(got_k), _bits(want_k)), (begin, end)
        assert np.array_equal(got_v, want_v), (begin, end)


@pytest.mark.parametrize("kind", ["f32", "f64"])
@pytest.mark.parametrize("descending", [False, True])
def test_radix_oracle_signed_zero_tie_every_window(kind, descending):
    """rccl-cub/src/ordering_backend/tests.rs:135-172 requires +0.0 and -0.0
    to have equal digits in every window (1 to 8 bits at every position) and
    in both orders. As a sort: a two-key input of opposite-signed zeros is a
    tie in every bit window, so a stable sort leaves it unchanged, whichever
    zero comes first. Without the collapse, some window separates them."""
    dt = np.dtype(NP[kind])
    width = 8 * dt.itemsize
    for first, second in ((0.0, -0.0), (-0.0, 0.0)):
        keys = np.array([first, second], dtype=dt)
        for begin in range(width):
            for end in range(begin + 1, min(width, begin + 8) + 1):
                got = oracle.radix_sort(kind, keys, None, descending, begin, end)
                assert np.array_equal(_bits(got), _bits(keys)), (first, begin, end)


def _ieee_total_order_tied_zeros(bits_a, bits_b, width):
    """IEEE 754-2008 totalOrder (section 5.10) with -0 and +0 tied: numbers by
    value (IEEE <); negative NaNs below every number and positive NaNs above;
    among NaNs of one sign, the larger payload lies further from zero."""
    import struct

    fmt = {32: ("<I", "<f"), 64: ("<Q", "<d")}[width]
    a = struct.unpack(fmt[1], struct.pack(fmt[0], bits_a))[0]
    b = struct.unpack(fmt[1], struct.pack(fmt[0], bits_b))[0]
    sign = 1 << (width - 1)

    def cls(bits, x):
        if x != x:
            return 0 if bits & sign else 2
        return 1

    ca, cb = cls(bits_a, a), cls(bits_b, b)
    if ca != cb:
        return -1 if ca < cb else 1
    if ca == 1:
        return -1 if a < b else (1 if a > b else 0)
    pa, pb = bits_a & (sign - 1), bits_b & (sign - 1)
    if ca == 0:  # negative NaNs: larger payload first
        pa, pb = pb, pa
    return -1 if pa < pb else (1 if pa > pb else 0)


@pytest.mark.parametrize("kind", ["f32", "f64"])
@pytest.mark.parametrize("descending", [False, True])
def test_radix_oracle_float_order_vs_python_sorted(kind, descending):
    """The float radix order is IEEE totalOrder with -0.0 and +0.0 tied, as a
    stable sort: checked against Python's stable sorted() under a comparator
    written from that definition (float comparisons for numbers, payload
    rules for NaN), on keys with many interleaved signed zeros, infinities,
    denormals, extremes and NaNs of both signs and several payloads."""
    import functools

    n = 6000
    dt = np.dtype(NP[kind])
    ut = BITS_OF[dt.itemsize]
    width = 8 * dt.itemsize
    keys = _special_float_keys(kind, n, 901 + width).copy()
    bits = keys.view(ut)
    rng = np.random.default_rng(77 + width)
    sign = ut(1) << ut(width - 1)
    exp_all = ut((1 << (width - 1)) - 1) ^ ut((1 << (23 if width == 32 else 52)) - 1)
    zpos = rng.integers(0, n, size=n // 5)
    bits[zpos] = np.where(rng.integers(0, 2, size=zpos.size) == 1, sign, ut(0)).astype(ut)
    npos = rng.integers(0, n, size=n // 50)
    payload = rng.integers(1, 4, size=npos.size).astype(ut)
    quiet = ut(1) << ut((22 if width == 32 else 51))
    nan_bits = exp_all | payload | np.where(rng.integers(0, 2, size=npos.size) == 1, quiet,
                                            ut(0)).astype(ut)
    bits[npos] = np.where(rng.integers(0, 2, size=npos.size) == 1, nan_bits | sign, nan_bits)
    idx = np.arange(n, dtype=np.uint32)
    cmp = functools.cmp_to_key(
        lambda i, j: _ieee_total_order_tied_zeros(int(bits[i]), int(bits[j]), width))
    want = sorted(range(n), key=cmp, reverse=descending)  # stable in both directions
    got_k, got_v = oracle.radix_sort(kind, keys, idx, descending)
    assert got_v.tolist() == want
    assert np.array_equal(_bits(got_k), bits[np.array(want)])


def test_radix_oracle_pairs_probe_family():
    # rccl-cub/examples/device_radix_sort_pairs_probe.rs:34-176: narrow key
    # domain, Rust's stable sort_by_key as the reference.
    idx = np.arange(10_003, dtype=np.uint64)
    h = (idx * np.uint64(2_654_435_761)) & np.uint64(0xFFFFFFFF)
    r = idx & np.uint64(31)
    rot = ((h << r) | (h >> ((np.uint64(32) - r) % np.uint64(32)))) & np.uint64(0xFFFFFFFF)
    keys = (rot & np.uint64(0x3FF)).astype(np.uint32)
    values = np.arange(keys.size, dtype=np.int32)
    pairs = list(zip(keys.tolist(), values.tolist()))
    asc = sorted(pairs, key=lambda p: p[0])
    desc = sorted(pairs, key=lambda p: -p[0])
    k, v = oracle.radix_sort("u32", keys, values)
    assert list(zip(k.tolist(), v.tolist())) == asc
    k, v = oracle.radix_sort("u32", keys, values, descending=True)
    assert list(zip(k.tolist(), v.tolist())) == desc
    k, v = oracle.radix_sort("u64", keys.astype(np.uint64), values.astype(np.uint64))
    assert list(zip(k.tolist(), v.tolist())) == asc
    # :255-305: bit window 0..24 sorts by the low 24 bits only.
    wk = (((np.arange(10_003, dtype=np.uint64) & np.uint64(0xFF)) << np.uint64(24)) |
          ((np.arange(10_003, dtype=np.uint64) * np.uint64(97)) & np.uint64(0x3FF))).astype(np.uint32)
    wv = np.arange(wk.size, dtype=np.int32)
    for d in (False, True):
        k, v = oracle.radix_sort("u32", wk, wv, d, 0, 24)
        exp = sorted(zip(wk.tolist(), wv.tolist()),
                     key=(lambda p: -(p[0] & 0xFFFFFF)) if d else (lambda p: p[0] & 0xFFFFFF))
        assert list(zip(k.tolist(), v.tolist())) == exp


# ---------------------------------------------------------------------------
# Merge and merge sort vs the standard library.
# ---------------------------------------------------------------------------
def _int_keys(kind, n, rng, domain):
    dt = np.dtype(NP[kind])
    lo = 0 if dt.kind == "u" else -domain // 2
    return rng.integers(lo, lo + domain, size=n).astype(dt)


@pytest.mark.parametrize("kind", ["u8", "i16", "u32", "i64", "f32", "f64"])
@pytest.mark.parametrize("descending", [False, True])
def test_merge_oracle_vs_heapq(kind, descending):
    rng = np.random.default_rng(3)
    for na, nb, domain in [(0, 0, 5), (0, 9, 5), (13, 0, 5), (500, 700, 20), (3000, 2000, 100)]:
        a = np.sort(_int_keys(kind, na, rng, domain), kind="stable")
        b = np.sort(_int_keys(kind, nb, rng, domain), kind="stable")
        if descending:
            a, b = a[::-1].copy(), b[::-1].copy()
        av = np.arange(na, dtype=np.uint32)
        bv = (np.arange(nb) | (1 << 31)).astype(np.uint32)
        want = list(heapq.merge(zip(a.tolist(), av.tolist()), zip(b.tolist(), bv.tolist()),
                                key=lambda p: p[0], reverse=descending))
        k, v = oracle.merge(kind, a, b, av, bv, descending)
        assert list(zip(k.tolist(), v.tolist())) == want


@pytest.mark.parametrize("kind", ["i8", "u16", "i32", "u64", "f32", "f64"])
@pytest.mark.parametrize("descending", [False, True])
def test_merge_sort_oracle_vs_sorted(kind, descending):
    rng = np.random.default_rng(5)
    for n, domain in [(0, 3), (1, 3), (2, 3), (1000, 10), (7000, 5000)]:
        keys = _int_keys(kind, n, rng, domain)
        vals = np.arange(n, dtype=np.uint64)
        want = sorted(zip(keys.tolist(), vals.tolist()), key=lambda p: p[0], reverse=descending)
        k, v = oracle.merge_sort(kind, keys, vals, descending)
        assert list(zip(k.tolist(), v.tolist())) == want
        assert np.array_equal(oracle.merge_sort(kind, keys, descending=descending), k)


# ---------------------------------------------------------------------------
# Set operations vs multiset algebra and a per-run value rule.
# ---------------------------------------------------------------------------
def _runs(keys, vals):
    """Group a sorted sequence into {key: [values in order]}."""
    out = collections.OrderedDict()
    for k, v in zip(keys, vals):
        out.setdefault(k, []).append(v)
    return out


def _set_by_runs(op, a, av, b, bv, descending):
    """For a key with m items in A and n in B: union keeps all m of A's then
    B's last n-m; intersection A's first min(m, n); difference A's last
    m-n; symmetric difference the longer side's last |m-n|. Keys come out in
    the sequence order (rccl-cub/src/ordering_backend/set.rs:564-827)."""
    ra, rb = _runs(a, av), _runs(b, bv)
    keys = sorted(set(ra) | set(rb), reverse=descending)
    ok, ov = [], []
    for k in keys:
        xa, xb = ra.get(k, []), rb.get(k, [])
        m, n = len(xa), len(xb)
        if op == "union":
            take = xa + xb[m:] if n > m else xa
        elif op == "intersection":
            take = xa[:min(m, n)]
        elif op == "difference":
            take = xa[n:] if m > n else []
        else:
            take = xa[n:] if m > n else xb[m:]
        ok += [k] * len(take)
        ov += take
    return ok, ov


@pytest.mark.parametrize("kind", ["u8", "i16", "i32", "u64", "f64"])
@pytest.mark.parametrize("op", OPS)
def test_set_oracle_vs_multiset_algebra(kind, op):
    rng = np.random.default_rng(11)
    for na, nb, domain in [(0, 0, 4), (0, 50, 4), (60, 0, 4), (700, 900, 12), (4000, 3000, 300)]:
        for descending in (False, True):
            a = np.sort(_int_keys(kind, na, rng, domain), kind="stable")
            b = np.sort(_int_keys(kind, nb, rng, domain), kind="stable")
            if descending:
                a, b = a[::-1].copy(), b[::-1].copy()
            av = np.arange(na, dtype=np.int32)
            bv = (np.arange(nb) + 1_000_000).astype(np.int32)
            k, v = oracle.set_op(op, kind, a, b, av, bv, descending)
            ca, cb = collections.Counter(a.tolist()), collections.Counter(b.tolist())
            counts = {"union": ca | cb, "intersection": ca & cb, "difference": ca - cb,
                      "symmetric_difference": (ca - cb) + (cb - ca)}[op]
            assert collections.Counter(k.tolist()) == counts
            wk, wv = _set_by_runs(op, a.tolist(), av.tolist(), b.tolist(), bv.tolist(), descending)
            assert k.tolist() == wk and v.tolist() == wv
            assert oracle.set_op(op, kind, a, b, descending=descending, count_only=True) == len(wk)


def test_set_oracle_reference_families():
    # rccl-thrust/examples/set_operations_tests.rs:491-590
    n = 25_000
    evens = (np.arange(n) * 2).astype(np.int32)
    odds = evens + 1
    assert np.array_equal(oracle.set_op("union", "i32", evens, odds),
                          np.arange(2 * n, dtype=np.int32))
    assert oracle.set_op("intersection", "i32", evens, odds).size == 0
    assert np.array_equal(oracle.set_op("union", "i32", evens, evens), evens)
    assert oracle.set_op("difference", "i32", evens, evens).size == 0
    first = sorted(((i * 37 + 11) % 13) - 6 for i in range(4097))
    second_all = sorted(((i * 29 + 7) % 13) - 6 for i in range(8194))
    for second_len in [0, 1, 2048, 4097, 4098, 8194]:
        second = second_all[:second_len]
        ca, cb = collections.Counter(first), collections.Counter(second)
        for op, c in [("union", ca | cb), ("intersection", ca & cb), ("difference", ca - cb),
                      ("symmetric_difference", (ca - cb) + (cb - ca))]:
            got = oracle.set_op(op, "i32", np.array(first, np.int32), np.array(second, np.int32))
            assert got.tolist() == sorted(c.elements())


def test_splitmix64_known_answer():
    # splitmix64 finaliser of state 0 (Steele, Lea and Flood 2014; the
    # constants of Java's SplittableRandom).
    assert oracle.splitmix64(0) == 0xE220A8397B1DCDAF


@pytest.mark.parametrize("n", [0, 1, 7, 1000, 65537, 1 << 20])
@pytest.mark.parametrize("threads", [1, 3, 8, 16])
def test_cpu_baseline_sorts_vs_numpy(n, threads):
    """The CPU baseline's comparison sorts (std::sort and the threaded
    chunk-sort + merge-path merges) against numpy's sort, with heavy
    duplicates so ties cross chunk and slice boundaries."""
    rng = np.random.default_rng(n * 31 + threads)
    keys = rng.integers(0, max(1, n // 8) + 1, size=n, dtype=np.uint64).astype(np.uint32)
    keys[: n // 3] = rng.integers(0, 1 << 32, size=n // 3, dtype=np.uint64).astype(np.uint32)
    want = np.sort(keys)
    assert np.array_equal(oracle.sort_unstable_u32(keys), want)
    assert np.array_equal(oracle.par_sort_unstable_u32(keys, threads), want)


@pytest.mark.parametrize("n", [0, 1, 7, 1000, 65537, 1 << 19])
@pytest.mark.parametrize("threads", [1, 3, 16])
def test_cpu_baseline_stable_pairs_vs_numpy(n, threads):
    """The stable pair sort substitute (one thread: std::stable_sort; more:
    chunk stable sorts + stable merge-path merges) against numpy's stable
    argsort, with heavy ties crossing chunk boundaries."""
    rng = np.random.default_rng(n * 7 + threads)
    keys = rng.integers(0, max(1, n // 16) + 1, size=n, dtype=np.uint64)
    keys[::5] = rng.integers(0, 1 << 63, size=keys[::5].size, dtype=np.uint64) << np.uint64(1)
    vals = np.arange(n, dtype=np.uint32)
    order = np.argsort(keys, kind="stable")
    gk, gv = oracle.stable_sort_pairs_u64_u32(keys, vals, threads)
    assert np.array_equal(gk, keys[order]) and np.array_equal(gv, vals[order])


def test_cpu_baseline_merge_and_set_ops_vs_oracle():
    """The std::merge / std::set_* substitutes agree with the oracle's
    restatements of the reference's merge and host_set_by."""
    rng = np.random.default_rng(5)
    a = np.sort(rng.integers(0, 500, size=4000).astype(np.uint32))
    b = np.sort(rng.integers(0, 500, size=3000).astype(np.uint32))
    av = np.arange(a.size, dtype=np.uint32)
    bv = np.arange(b.size, dtype=np.uint32) | np.uint32(1 << 31)
    gk, gv = oracle.merge_pairs_u32(a, av, b, bv)
    wk, wv = oracle.merge("u32", a, b, av, bv)
    assert np.array_equal(gk, wk) and np.array_equal(gv, wv)
    a64, b64 = a.astype(np.uint64) * np.uint64(1 << 33), b.astype(np.uint64) * np.uint64(1 << 33)
    for op in ("union", "intersection", "difference", "symmetric_difference"):
        assert np.array_equal(oracle.std_set_op_u64(op, a64, b64),
                              oracle.set_op(op, "u64", a64, b64))


def _reference_rows(arity, n):
    """The row generator of rccl-thrust/examples/record_sort.rs:11-23."""
    idx = np.arange(n, dtype=np.int64)[:, None]
    col = np.arange(arity, dtype=np.int64)[None, :]
    return ((idx * (col * 6 + 5) + col * 3) % (11 + col * 2)).astype(np.uint32)


@pytest.mark.parametrize("arity", [2, 3, 4, 5, 6])
@pytest.mark.parametrize("n", [0, 1, 31, 257, 10003])
def test_record_sort_oracle_vs_lexsort(arity, n):
    """Row sort against numpy's stable lexsort (last key primary) on the
    reference's row generator and on random rows over a small alphabet, with
    the input index as payload so stability is visible."""
    rng = np.random.default_rng(arity * 1000 + n)
    for rows in (_reference_rows(arity, n),
                 rng.integers(0, 3, size=(n, arity), dtype=np.uint64).astype(np.uint32),
                 rng.integers(0, 1 << 32, size=(n, arity), dtype=np.uint64).astype(np.uint32)):
        pay = np.arange(n, dtype=np.uint64)
        order = np.lexsort(rows.T[::-1]) if n else np.arange(0)
        out_rows, out_pay = oracle.record_sort(rows, pay)
        assert np.array_equal(out_rows, rows[order])
        assert np.array_equal(out_pay, pay[order])


def test_record_sort_oracle_rejects_arity():
    with pytest.raises(ValueError):
        oracle.record_sort(np.zeros((3, 1), dtype=np.uint32))
    with pytest.raises(ValueError):
        oracle.record_sort(np.zeros((3, 7), dtype=np.uint32))


# ---------------------------------------------------------------------------
# Adjacent-run compactions vs an itertools.groupby restatement
# (rccl-cub/src/compaction_kernels.rs:64-236, grouped_reduction.rs:17-75).
# ---------------------------------------------------------------------------
def _groupby_reduce(keys, vals, op):
    import itertools
    out_k, out_v = [], []
    idx = 0
    for key, grp in itertools.groupby(keys.tolist() if keys.ndim == 1 else
                                      [tuple(r) for r in keys.tolist()]):
        n = len(list(grp))
        run = vals[idx:idx + n].tolist()
        idx += n
        if op == "natural_bag_add":
            agg = run[0]
            for v in run[1:]:
                agg = (agg + v) % (1 << 64)
        elif op == "boolean_or":
            agg = run[0]
            for v in run[1:]:
                agg = 1 if (agg or v) else 0
        else:
            agg = run[0]
            for v in run[1:]:
                agg = min(max(agg + v - agg * v, 0.0), 1.0)
        out_k.append(key)
        out_v.append(agg)
    return out_k, out_v


@pytest.mark.parametrize("op", ["natural_bag_add", "boolean_or", "independent_probability_or"])
def test_reduce_by_key_oracle_vs_groupby(op):
    rng = np.random.default_rng(11)
    for n in (0, 1, 2, 31, 257, 5000):
        keys = np.sort(rng.integers(0, max(1, n // 4), size=n)).astype(np.int32)
        vals = {"natural_bag_add": rng.integers(0, 2**64, size=n, dtype=np.uint64),
                "boolean_or": rng.integers(0, 2, size=n).astype(np.uint8),
                "independent_probability_or": rng.random(n)}[op]
        exp_k, exp_v = _groupby_reduce(keys, vals, op)
        out_k, out_v = oracle.reduce_by_key(keys, vals, op, "i32")
        assert out_k.tolist() == exp_k
        assert out_v.tolist() == exp_v  # Python floats fold without fused multiply-add
    # Rows: a run is a run of equal rows.
    rows = np.repeat(rng.integers(0, 3, size=(400, 3)).astype(np.uint32), 3, axis=0)
    vals = rng.integers(0, 100, size=len(rows), dtype=np.uint64)
    exp_k, exp_v = _groupby_reduce(rows, vals, "natural_bag_add")
    out_k, out_v = oracle.reduce_by_key(rows, vals, "natural_bag_add")
    assert [tuple(r) for r in out_k.tolist()] == exp_k and out_v.tolist() == exp_v


def test_unique_oracle_vs_groupby():
    import itertools
    rng = np.random.default_rng(12)
    for n in (0, 1, 31, 32, 33, 255, 256, 257, 513):
        keys = (np.arange(n) // 3).astype(np.uint32)  # examples/compaction.rs:117-146
        assert oracle.unique(keys, "u32").tolist() == [k for k, _ in itertools.groupby(keys)]
    f = np.array([0.0, -0.0, np.nan, np.nan, 1.0, 1.0], dtype=np.float64)
    # IEEE ==: -0 joins the run of +0, NaN never joins a run.
    assert oracle.unique(f, "f64").view(np.uint64).tolist() == \
        f[[0, 2, 3, 4]].view(np.uint64).tolist()
    rows = rng.integers(0, 2, size=(1000, 2)).astype(np.uint32)
    exp = [k for k, _ in itertools.groupby([tuple(r) for r in rows.tolist()])]
    assert [tuple(r) for r in oracle.unique(rows).tolist()] == exp


def test_probability_or_known_answers():
    """rccl-cub/src/grouped_reduction.rs:209-224."""
    import struct
    second = oracle.prob_or(oracle.prob_or(0.1, 0.2), 0.3)
    assert struct.unpack("<Q", struct.pack("<d", second))[0] == 4_602_606_761_578_608_985
    assert oracle.prob_or(1.0, 0.5) == 1.0
