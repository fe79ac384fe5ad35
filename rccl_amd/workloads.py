"""Seeded synthetic inputs for the five benchmark configurations.

Every value is a pure function of (seed, index) through splitmix64, so the GPU
run and the CPU checker see identical data without shipping any. Seeds are
fixed here; the config text each generator implements is quoted in its
docstring, and where that text is ambiguous the reading chosen is stated.
"""
from __future__ import annotations

import numpy as np

SEEDS = {
    "C1": 0x0C1_5EED,
    "M32": 0x3232_5EED,
    "M64": 0x6464_5EED,
    "C2": 0x0C2_5EED,
    "C2_dict": 0x0C2D_1C7,
    "C2_zipf": 0x0C2_21F,
    "C3": 0x0C3_5EED,
    "C3_pos": 0x0C3_9051,
    "C4a": 0x0C4A_5EED,
    "C4b": 0x0C4B_5EED,
    "C4c": 0x0C4C_5EED,
    "C5_pool": 0x0C5_9001,
    "C5a": 0x0C5A_5EED,
    "C5b": 0x0C5B_5EED,
}

_U64 = np.uint64
_CHUNK = 1 << 24


def splitmix64(x: np.ndarray) -> np.ndarray:
    """splitmix64 finaliser applied elementwise to uint64 states."""
    out = np.array(x, dtype=_U64, copy=True)
    _splitmix64_inplace(out, np.empty_like(out))
    return out


def _splitmix64_inplace(x: np.ndarray, tmp: np.ndarray) -> None:
    # In place over preallocated buffers: fresh temporaries per operation
    # would cost more in first-touch page faults than the arithmetic.
    with np.errstate(over="ignore"):
        np.add(x, _U64(0x9E3779B97F4A7C15), out=x)
        for shift, mult in ((30, 0xBF58476D1CE4E5B9), (27, 0x94D049BB133111EB)):
            np.right_shift(x, _U64(shift), out=tmp)
            np.bitwise_xor(x, tmp, out=x)
            np.multiply(x, _U64(mult), out=x)
        np.right_shift(x, _U64(31), out=tmp)
        np.bitwise_xor(x, tmp, out=x)


def hash_range(seed: int, n: int, start: int = 0) -> np.ndarray:
    """splitmix64(seed + i) for i in [start, start + n), as uint64."""
    out = np.empty(n, dtype=_U64)
    if n == 0:
        return out
    base = np.arange(min(n, _CHUNK), dtype=_U64)
    tmp = np.empty(min(n, _CHUNK), dtype=_U64)
    for lo in range(0, n, _CHUNK):
        hi = min(n, lo + _CHUNK)
        x = out[lo:hi]
        with np.errstate(over="ignore"):
            np.add(base[:hi - lo], _U64((seed + start + lo) & 0xFFFFFFFFFFFFFFFF), out=x)
        _splitmix64_inplace(x, tmp[:hi - lo])
    return out


def uniform_u32(n: int, seed: int) -> np.ndarray:
    """key[i] = high 32 bits of splitmix64(seed + i): uniform over 32 bits."""
    return (hash_range(seed, n) >> _U64(32)).astype(np.uint32)


def c1_keys(n: int = 1 << 20) -> np.ndarray:
    """C1: 2^20 u32 keys uniform over the full 32-bit range from a fixed seed."""
    return uniform_u32(n, SEEDS["C1"])


def metric_u32_keys(n: int = 1 << 28) -> np.ndarray:
    """Metric workload: 2^28 uniform u32 keys."""
    return uniform_u32(n, SEEDS["M32"])


def c2_uniform(n: int = 1 << 26, seed: int | None = None):
    """C2 uniform: u64 keys uniform over 64 bits, value = original index (u32)."""
    keys = hash_range(SEEDS["C2"] if seed is None else seed, n)
    return keys, np.arange(n, dtype=np.uint32)


def c2_low_entropy(n: int = 1 << 26):
    """C2 low-entropy: 256 distinct random u64 values with Zipf s=1.1
    frequencies; value = original index. u_i = 53-bit uniform from
    splitmix64, key = D[inverse CDF(u_i)]."""
    dictionary = hash_range(SEEDS["C2_dict"], 256)
    weights = (np.arange(1, 257, dtype=np.float64)) ** -1.1
    cdf = np.cumsum(weights / weights.sum())
    cdf[-1] = 1.0
    keys = np.empty(n, dtype=_U64)
    for lo in range(0, n, _CHUNK):
        hi = min(n, lo + _CHUNK)
        u = (hash_range(SEEDS["C2_zipf"], hi - lo, lo) >> _U64(11)).astype(np.float64) * 2.0**-53
        idx = np.searchsorted(cdf, u, side="right")
        keys[lo:hi] = dictionary[np.minimum(idx, 255)]
    return keys, np.arange(n, dtype=np.uint32)


def metric_pairs(n: int = 1 << 28):
    """Metric workload: u64 keys uniform over 64 bits with u32 index values."""
    return c2_uniform(n, SEEDS["M64"])


def c3_special_counts(n: int) -> dict:
    """Exact special-value counts for C3 at size n."""
    zeros = n // 100
    infs = n // 1000
    return {
        "+0": zeros,
        "-0": zeros,
        "+inf": infs // 2,
        "-inf": infs - infs // 2,
        "denormal": n // 1000,
        "nan": n // 10000,
    }


def c3_keys(n: int = 1 << 28) -> np.ndarray:
    """C3: f32 keys ~ N(0, 1e3) (read as sigma = 1e3), with 1% +0.0, 1% -0.0,
    0.1% +-inf (half each), 0.1% denormals (random sign, mantissa in
    [1, 2^23-1]) and 0.01% quiet NaN (0x7fc00000, positive) at seeded
    distinct positions. Base values come from Box-Muller on two 53-bit
    uniforms per index, in float64 rounded to float32."""
    seed = SEEDS["C3"]
    out = np.empty(n, dtype=np.float32)
    for lo in range(0, n, _CHUNK):
        hi = min(n, lo + _CHUNK)
        idx = np.arange(lo, hi, dtype=_U64)
        with np.errstate(over="ignore"):
            a = splitmix64(idx * _U64(2) + _U64(seed))
            b = splitmix64(idx * _U64(2) + _U64(seed + 1))
        u1 = ((a >> _U64(11)).astype(np.float64) + 1.0) * 2.0**-53  # (0, 1]
        u2 = (b >> _U64(11)).astype(np.float64) * 2.0**-53
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
        out[lo:hi] = (1000.0 * z).astype(np.float32)
    bits = out.view(np.uint32)
    counts = c3_special_counts(n)
    total = sum(counts.values())
    prio = hash_range(SEEDS["C3_pos"], n)
    chosen = np.argpartition(prio, total - 1)[:total] if total < n else np.arange(n)
    chosen = chosen[np.argsort(prio[chosen], kind="stable")]
    pos = 0
    sel = {}
    for name in ("+0", "-0", "+inf", "-inf", "denormal", "nan"):
        sel[name] = chosen[pos:pos + counts[name]]
        pos += counts[name]
    bits[sel["+0"]] = 0x00000000
    bits[sel["-0"]] = 0x80000000
    bits[sel["+inf"]] = 0x7F800000
    bits[sel["-inf"]] = 0xFF800000
    d = hash_range(SEEDS["C3_pos"] ^ 0xDE40, counts["denormal"])
    mant = (d % _U64((1 << 23) - 1)).astype(np.uint32) + np.uint32(1)
    sign = ((d >> _U64(63)).astype(np.uint32)) << np.uint32(31)
    bits[sel["denormal"]] = sign | mant
    bits[sel["nan"]] = 0x7FC00000
    return out


def _sorted_u32_24bit(n: int, seed: int) -> np.ndarray:
    """The n values (splitmix64(seed + i) >> 40) in ascending order, built by
    counting (the values lie in [0, 2^24))."""
    counts = np.zeros(1 << 24, dtype=np.int64)
    for lo in range(0, n, _CHUNK):
        part = (hash_range(seed, min(n, lo + _CHUNK) - lo, lo) >> _U64(40)).astype(np.int64)
        counts += np.bincount(part, minlength=1 << 24)
    return np.repeat(np.arange(1 << 24, dtype=np.uint32), counts)


def c4_merge_inputs(n_each: int = 1 << 27):
    """C4 merge: two independently generated ascending-sorted u32 arrays with
    values in [0, 2^24) (heavy duplicates). Payloads: A[i] -> i,
    B[i] -> i | 0x80000000, so the source of every output is observable."""
    a = _sorted_u32_24bit(n_each, SEEDS["C4a"])
    b = _sorted_u32_24bit(n_each, SEEDS["C4b"])
    pa = np.arange(n_each, dtype=np.uint32)
    pb = np.arange(n_each, dtype=np.uint32) | np.uint32(0x80000000)
    return a, pa, b, pb


def c4_merge_sort_keys(n: int = 1 << 26) -> np.ndarray:
    """C4 merge sort: unsorted u32 keys from the same [0, 2^24) value range."""
    return (hash_range(SEEDS["C4c"], n) >> _U64(40)).astype(np.uint32)


def _c5_side(pool: np.ndarray, seed: int, n: int) -> np.ndarray:
    half = n // 2
    prio = hash_range(seed, pool.size)
    from_pool = pool[np.argpartition(prio, half - 1)[:half]] if half < pool.size else pool.copy()
    fresh = hash_range(seed ^ 0xF2E5, n - half)
    side = np.sort(np.concatenate([from_pool, fresh]))
    # About 10% of positions start a run of 2-4 copies of their key, which
    # overwrite the following positions; the size stays n.
    h = hash_range(seed ^ 0xD0B1, n)
    src = np.nonzero(h % _U64(100) < _U64(10))[0]
    reps = (2 + (h[src] >> _U64(32)) % _U64(3)).astype(np.int64)
    for k in (1, 2, 3):
        m = (k < reps) & (src + k < n)
        side[src[m] + k] = side[src[m]]
    return np.sort(side)


def c5_inputs(n_each: int = 1 << 26):
    """C5: sorted u64 multisets A and B of n_each items. A shared pool of
    n_each seeded keys; each side takes a seeded n_each/2 subset of the pool
    plus n_each/2 fresh keys of its own (the config's "2^25 fresh keys
    unique to each"); then about 10% of positions are duplicated 2-4x with
    the size held at n_each; both sorted ascending."""
    pool = hash_range(SEEDS["C5_pool"], n_each)
    a = _c5_side(pool, SEEDS["C5a"], n_each)
    b = _c5_side(pool, SEEDS["C5b"], n_each)
    return a, b


def record_rows(arity: int, n: int) -> np.ndarray:
    """Relation rows of the reference's record-sort example and benchmark
    (rccl-thrust/examples/record_sort.rs:11-23, record_sort_benchmark.rs:33-39):
    row[i][c] = (i * (6c + 5) + 3c) mod (11 + 2c), an (n, arity) u32 array."""
    idx = np.arange(n, dtype=np.uint64)[:, None]
    col = np.arange(arity, dtype=np.uint64)[None, :]
    return ((idx * (col * _U64(6) + _U64(5)) + col * _U64(3)) % (_U64(11) + col * _U64(2))).astype(
        np.uint32)


RECORD_SORT_ROWS = (1 << 20) + 13  # record_sort_benchmark.rs:4


REFERENCE_BENCH_SEED = 0x534D4152545F534F


def reference_bench_u32(n: int = 1 << 24) -> np.ndarray:
    """Keys of the reference's radix-sort benchmark (benchmarks/ordering-reference.cu:23-33,
    the input of its published 2^24 u32 figure): x = i ^ 0x534d4152545f534f, then the
    xorshift steps x ^= x << 13, x ^= x >> 7, x ^= x << 17 in 64-bit arithmetic, and the
    key is the low 32 bits of x."""
    x = np.arange(n, dtype=np.uint64) ^ _U64(REFERENCE_BENCH_SEED)
    x ^= x << _U64(13)
    x ^= x >> _U64(7)
    x ^= x << _U64(17)
    return x.astype(np.uint32)
