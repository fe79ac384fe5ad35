"""Device-resident versions of the benchmark inputs in rccl_amd.workloads.

Each generator returns torch tensors on the GPU holding exactly the bits the
host generator of the same name returns (uint64 data is held in int64
tensors, uint32 in int32). The splitmix64 arithmetic runs in wrapping int64;
right shifts are made logical by masking. Producing the inputs where they are
consumed keeps the benchmark's set-up to seconds at 2^28 items.
"""
from __future__ import annotations

import torch

from .workloads import SEEDS

_C0 = 0x9E3779B97F4A7C15
_C1 = 0xBF58476D1CE4E5B9
_C2 = 0x94D049BB133111EB
_SIGN = -(1 << 63)


def _signed(u: int) -> int:
    u &= (1 << 64) - 1
    return u - (1 << 64) if u >= (1 << 63) else u


def shr(x: torch.Tensor, k: int) -> torch.Tensor:
    """Logical right shift of int64 bit patterns."""
    return (x >> k) & ((1 << (64 - k)) - 1)


def splitmix64(x: torch.Tensor) -> torch.Tensor:
    x = x + _signed(_C0)
    x = (x ^ shr(x, 30)) * _signed(_C1)
    x = (x ^ shr(x, 27)) * _signed(_C2)
    return x ^ shr(x, 31)


def hash_range(seed: int, n: int, start: int = 0, device="cuda") -> torch.Tensor:
    """splitmix64(seed + i) for i in [start, start + n) as int64 bit patterns."""
    idx = torch.arange(n, dtype=torch.int64, device=device)
    return splitmix64(idx + _signed(seed + start))


def _u64_mod(x: torch.Tensor, m: int) -> torch.Tensor:
    """Unsigned x mod m for int64 bit patterns (m < 2^31)."""
    hi, lo = shr(x, 32), x & 0xFFFFFFFF
    return ((hi % m) * ((1 << 32) % m) + lo % m) % m


def sort_u64(x: torch.Tensor) -> torch.Tensor:
    """Ascending unsigned order of int64 bit patterns."""
    return torch.sort(x ^ _SIGN).values ^ _SIGN


def c1_keys(n: int = 1 << 20, device="cuda") -> torch.Tensor:
    return shr(hash_range(SEEDS["C1"], n, device=device), 32).to(torch.int32)


def metric_u32_keys(n: int = 1 << 28, device="cuda") -> torch.Tensor:
    return shr(hash_range(SEEDS["M32"], n, device=device), 32).to(torch.int32)


def metric_pairs(n: int = 1 << 28, device="cuda"):
    keys = hash_range(SEEDS["M64"], n, device=device)
    return keys, torch.arange(n, dtype=torch.int32, device=device)


def c2_uniform(n: int = 1 << 26, device="cuda"):
    keys = hash_range(SEEDS["C2"], n, device=device)
    return keys, torch.arange(n, dtype=torch.int32, device=device)


def c2_low_entropy(n: int = 1 << 26, device="cuda"):
    """Device twin of workloads.c2_low_entropy (bit-identical: the uniforms are
    exact 53-bit values and the inverse CDF is a comparison search over the
    same float64 table)."""
    import numpy as np

    dictionary = hash_range(SEEDS["C2_dict"], 256, device=device)
    weights = np.arange(1, 257, dtype=np.float64) ** -1.1
    cdf_h = np.cumsum(weights / weights.sum())
    cdf_h[-1] = 1.0
    cdf = torch.from_numpy(cdf_h).to(device)
    u = shr(hash_range(SEEDS["C2_zipf"], n, device=device), 11).to(torch.float64) * 2.0 ** -53
    idx = torch.searchsorted(cdf, u, right=True).clamp_(max=255)
    del u
    return dictionary[idx], torch.arange(n, dtype=torch.int32, device=device)


def c3_keys(n: int = 1 << 28, device="cuda") -> torch.Tensor:
    """Device twin of workloads.c3_keys, as float32. The special values and
    their positions are bit-identical to the host generator's; the Box-Muller
    normals are computed with the device's float64 log/sqrt/cos, which may
    differ from the host libm in the last float64 place, and so (rarely) in
    the last float32 place of a normal value."""
    import math

    seed = SEEDS["C3"]
    out = torch.empty(n, dtype=torch.float32, device=device)
    chunk = 1 << 24
    for lo in range(0, n, chunk):
        hi = min(n, lo + chunk)
        idx = torch.arange(lo, hi, dtype=torch.int64, device=device)
        a = splitmix64(idx * 2 + _signed(seed))
        b = splitmix64(idx * 2 + _signed(seed + 1))
        u1 = (shr(a, 11).to(torch.float64) + 1.0) * 2.0 ** -53
        u2 = shr(b, 11).to(torch.float64) * 2.0 ** -53
        z = torch.sqrt(-2.0 * torch.log(u1)) * torch.cos(2.0 * math.pi * u2)
        out[lo:hi] = (1000.0 * z).to(torch.float32)
    bits = out.view(torch.int32)
    from .workloads import c3_special_counts

    counts = c3_special_counts(n)
    total = sum(counts.values())
    prio = hash_range(SEEDS["C3_pos"], n, device=device)
    # The `total` positions of smallest unsigned priority, in priority order.
    chosen = torch.sort(prio ^ _SIGN).indices[:total]
    del prio
    pos = 0
    sel = {}
    for name in ("+0", "-0", "+inf", "-inf", "denormal", "nan"):
        sel[name] = chosen[pos:pos + counts[name]]
        pos += counts[name]
    bits[sel["+0"]] = 0
    bits[sel["-0"]] = _signed32(0x80000000)
    bits[sel["+inf"]] = 0x7F800000
    bits[sel["-inf"]] = _signed32(0xFF800000)
    d = hash_range(SEEDS["C3_pos"] ^ 0xDE40, counts["denormal"], device=device)
    mant = _u64_mod(d, (1 << 23) - 1) + 1
    sign = shr(d, 63) << 31
    bits[sel["denormal"]] = _u32_bits(sign | mant)
    bits[sel["nan"]] = 0x7FC00000
    return out


def _sorted_u32_24bit(n: int, seed: int, device) -> torch.Tensor:
    v = shr(hash_range(seed, n, device=device), 40)
    counts = torch.bincount(v, minlength=1 << 24)
    return torch.repeat_interleave(torch.arange(1 << 24, dtype=torch.int32, device=device),
                                   counts, output_size=n)


def c4_merge_inputs(n_each: int = 1 << 27, device="cuda"):
    a = _sorted_u32_24bit(n_each, SEEDS["C4a"], device)
    b = _sorted_u32_24bit(n_each, SEEDS["C4b"], device)
    pa = torch.arange(n_each, dtype=torch.int32, device=device)
    pb = pa | _signed32(0x80000000)
    return a, pa, b, pb


def _u32_bits(v: torch.Tensor) -> torch.Tensor:
    """int32 bit patterns of int64 values in [0, 2^32)."""
    return (v - (v >= (1 << 31)).to(torch.int64) * (1 << 32)).to(torch.int32)


def _signed32(u: int) -> int:
    return u - (1 << 32) if u >= (1 << 31) else u


def c4_merge_sort_keys(n: int = 1 << 26, device="cuda") -> torch.Tensor:
    return shr(hash_range(SEEDS["C4c"], n, device=device), 40).to(torch.int32)


def _c5_side(pool: torch.Tensor, seed: int, n: int, device) -> torch.Tensor:
    half = n // 2
    prio = hash_range(seed, pool.numel(), device=device)
    if half < pool.numel():
        idx = torch.sort(prio ^ _SIGN).indices[:half]
        from_pool = pool[idx]
    else:
        from_pool = pool.clone()
    fresh = hash_range(seed ^ 0xF2E5, n - half, device=device)
    side = sort_u64(torch.cat([from_pool, fresh]))
    h = hash_range(seed ^ 0xD0B1, n, device=device)
    src = torch.nonzero(_u64_mod(h, 100) < 10).flatten()
    reps = 2 + shr(h[src], 32) % 3
    for k in (1, 2, 3):
        m = (reps > k) & (src + k < n)
        s = src[m]
        side[s + k] = side[s]
    return sort_u64(side)


def c5_inputs(n_each: int = 1 << 26, device="cuda"):
    pool = hash_range(SEEDS["C5_pool"], n_each, device=device)
    return _c5_side(pool, SEEDS["C5a"], n_each, device), _c5_side(pool, SEEDS["C5b"], n_each,
                                                                   device)


def record_rows(arity: int, n: int, device="cuda") -> torch.Tensor:
    """Device twin of workloads.record_rows, flattened row-major as int32."""
    idx = torch.arange(n, dtype=torch.int64, device=device)[:, None]
    col = torch.arange(arity, dtype=torch.int64, device=device)[None, :]
    return ((idx * (col * 6 + 5) + col * 3) % (11 + col * 2)).to(torch.int32).reshape(-1)
