#!/usr/bin/env python3
"""Benchmark of the ordering hot path on one MI355X.

Metric: Gkeys/s radix sort at 2^28 for u32 keys (the headline
``value``) and for u64-key/u32-value pairs (reported under ``pairs``), with the
fraction of the 8 TB/s HBM roofline. The C4 merge / merge sort and C5 set
operation shapes, and the reference's record-sort benchmark, are reported
under ``ordering``.

A step is one full pass of the operation over the resident input. Radix sort
is in place, so before every step its input is restored from a pristine
device copy; that copy is outside the HIP-event interval that times the sort
(``ms_per_step``) and inside the wall-clock interval (``ms_per_step_wall``).
Per-launch kernel durations come from the library's own hipEvent timing
(rccl_hip_timing_enable), recorded on the launch stream during the timed
steps. Inputs are generated on the device (rccl_amd.workloads_device, bit-
identical to the host generators the tests use).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "Gkeys/s radix sort (u32 keys; u64+u32 pairs) at 2^28; % of HBM roofline"


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _sorted_equal(torch, out, src):
    """Exact check: `out` equals `src` sorted ascending in unsigned order
    (torch.sort through a flipped sign bit), word for word; `src` and `out`
    are int32 or int64 storage of u32 or u64 keys."""
    sign = torch.tensor(-(1 << (8 * src.element_size() - 1)), dtype=src.dtype,
                        device=src.device)
    want = torch.sort(src ^ sign).values ^ sign
    return bool(torch.equal(out, want))


def _nondecreasing(torch, t, bits):
    """True if the unsigned view of t is non-decreasing."""
    if t.numel() < 2:
        return True
    if bits == 32:
        u = t.to(torch.int64) & 0xFFFFFFFF
        return bool((u[1:] >= u[:-1]).all().item())
    s = t ^ torch.tensor(-(1 << 63), dtype=torch.int64, device=t.device)
    return bool((s[1:] >= s[:-1]).all().item())


def _buffer(torch, DeviceBuffer, t, np_dtype):
    """Wrap a device tensor (same-width signed storage) as a DeviceBuffer."""
    return DeviceBuffer(t.contiguous(), np_dtype, t.numel())


def time_steps(torch, abi, stream, steps, warmup, step, before=None):
    """Run `step` warmup times, then `steps` timed times, then `steps` more
    with the library's per-launch timing on. Returns a dict: "ms" (median of
    the per-step hipEvent times, the reference's protocol), "mean", "min",
    "wall" (wall-clock ms per step, `before` included), "kernel_ms" ({kernel:
    mean ms per launch}), "launches" ({kernel: launches per step}) and
    "per_step" ([[(kernel, ms), ...] per profiled step]). The timed steps run
    without per-launch events, so ``ms`` carries no timing overhead."""
    for _ in range(warmup):
        if before:
            before()
        step()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for k in range(steps):
        if before:
            before()
        starts[k].record(stream)
        step()
        ends[k].record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    step_ms = sorted(s.elapsed_time(e) for s, e in zip(starts, ends))
    abi.timing_read()
    abi.timing_enable(True)
    per_step = []
    for _ in range(steps):
        if before:
            before()
        step()
        torch.cuda.synchronize()
        per_step.append([(name, kms) for name, kms, _items in abi.timing_read()])
    abi.timing_enable(False)
    per = {}
    for launches in per_step:
        for name, kms in launches:
            per.setdefault(name, []).append(kms)
    mid = len(step_ms) // 2
    median = step_ms[mid] if len(step_ms) % 2 else 0.5 * (step_ms[mid - 1] + step_ms[mid])
    return {"ms": median, "mean": sum(step_ms) / steps, "min": step_ms[0],
            "wall": (t1 - t0) * 1e3 / steps,
            "kernel_ms": {k: sum(v) / len(v) for k, v in per.items()},
            "launches": {k: len(v) // steps for k, v in per.items()}, "per_step": per_step}


def _steps(*args, **kw):
    """time_steps as (median ms, min ms, wall ms, kernel_ms, launches,
    per_step)."""
    t = time_steps(*args, **kw)
    return t["ms"], t["min"], t["wall"], t["kernel_ms"], t["launches"], t["per_step"]


def roofline(bytes_per_launch, launch_ms, kernel, traffic=None):
    achieved = bytes_per_launch / (launch_ms * 1e-3) / 1e9
    extra = {} if traffic is None else {
        "traffic_source": "profiles/hbm_traffic_bench_legs.txt (rocprofv3 FETCH_SIZE and "
                          "WRITE_SIZE, each scaled so a 1 GiB copy reads as 1 GiB)"}
    return {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "kernel": kernel,
        **extra,
    }


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "hbm_traffic_bench_legs.txt")


def profiled_traffic(kernel, log2n):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC
    summary (FETCH_SIZE and WRITE_SIZE scaled by a copy kernel of known size),
    or None when that summary does not cover this problem size (the summary
    is of the default run, whose sizes all derive from --log2n 28). A row is
    `name kernel... calls read write traffic algorithmic ratio`; the kernel
    label may hold spaces, so the traffic is read from the right."""
    if log2n != 28 or not os.path.exists(TRAFFIC_PROFILE):
        return None
    with open(TRAFFIC_PROFILE) as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 8 and parts[0] == kernel:
                return int(parts[-3])
    return None


def _rounded(d):
    return {k: round(v, 4) for k, v in d.items()}


# ---------------------------------------------------------------------------
# Radix sort legs (the metric).
# ---------------------------------------------------------------------------
def _check_stable_pairs(torch, src_keys, out_keys, out_vals, bits):
    """Exact check of a stable ascending sort of unsigned keys (same-width
    signed tensors) whose values are their original indices: keys
    non-decreasing, values a permutation, each value's key equal to its own
    key in the input, and indices rising within every run of equal keys."""
    n = src_keys.numel()
    if not _nondecreasing(torch, out_keys, bits):
        return False
    idx = out_vals.to(torch.int64) & 0xFFFFFFFF
    if not torch.equal(torch.sort(idx).values, torch.arange(n, device=idx.device)):
        return False
    if not torch.equal(src_keys[idx], out_keys):
        return False
    same = out_keys[1:] == out_keys[:-1]
    return bool((idx[1:] > idx[:-1])[same].all().item())


def _check_f32_descending(torch, src_bits, out_bits):
    """Exact check of a descending f32 radix sort (int32 bit views): the same
    multiset of bit patterns; positive NaNs first, then numbers non-increasing
    under IEEE compare, then negative NaNs; the signed zeros in input order."""
    if not torch.equal(torch.sort(out_bits).values, torch.sort(src_bits).values):
        return False
    out = out_bits.view(torch.float32)
    nan = torch.isnan(out)
    neg = out_bits < 0
    pos_nan, neg_nan = int((nan & ~neg).sum()), int((nan & neg).sum())
    n = out.numel()
    if not bool(nan[:pos_nan].all()) or not bool(nan[n - neg_nan:].all()):
        return False
    mid = out[pos_nan:n - neg_nan]
    if bool(torch.isnan(mid).any()) or not bool((mid[1:] <= mid[:-1]).all()):
        return False
    zo, zs = (out_bits & 0x7FFFFFFF) == 0, (src_bits & 0x7FFFFFFF) == 0
    return bool(torch.equal(out_bits[zo], src_bits[zs]))


def run_radix(torch, np, cub, abi, DeviceBuffer, keys_t, values_t, steps, warmup, kdt=None,
              descending=False):
    """In-place radix sort of a device-resident input, restored from a
    pristine copy before every step (outside the timed interval). Keys are
    u32/u64 (or kdt), values u32 original indices or None."""
    n = keys_t.numel()
    launch = cub.Program.load(0).on(torch.cuda.current_stream(0))
    if kdt is None:
        kdt = np.uint32 if keys_t.dtype == torch.int32 else np.uint64
    pristine_k = keys_t
    keys = _buffer(torch, DeviceBuffer, torch.empty_like(keys_t), kdt)
    if values_t is not None:
        pristine_v = values_t
        values = _buffer(torch, DeviceBuffer, torch.empty_like(values_t), np.uint32)
        ws = cub.device_radix_sort_pairs_workspace(launch, kdt, np.uint32, n)
    else:
        ws = cub.device_radix_sort_workspace(launch, kdt, n)

    def restore():
        keys.tensor.copy_(pristine_k)
        if values_t is not None:
            values.tensor.copy_(pristine_v)

    def sort():
        if values_t is not None:
            (cub.device_radix_sort_pairs_descending if descending
             else cub.device_radix_sort_pairs)(launch, keys, values, ws)
        else:
            (cub.device_radix_sort_keys_descending if descending
             else cub.device_radix_sort_keys)(launch, keys, ws)

    t = time_steps(torch, abi, launch.stream(), steps, warmup, sort, restore)
    bits = 8 * np.dtype(kdt).itemsize
    if np.dtype(kdt) == np.float32 and descending and values_t is None:
        ok = _check_f32_descending(torch, pristine_k, keys.tensor)
    elif values_t is not None and not descending and np.dtype(kdt).kind == "u":
        ok = _check_stable_pairs(torch, pristine_k, keys.tensor, values.tensor, bits)
    else:
        ok = _sorted_equal(torch, keys.tensor, pristine_k)
    return {"n": n, "ms": t["ms"], "ms_mean": t["mean"], "ms_min": t["min"], "ms_wall": t["wall"],
            "kernel_ms": t["kernel_ms"], "launches": t["launches"], "validated": bool(ok)}


def radix_leg(r, n, workload, key_bytes_model, pass_bytes, kernel_desc, traffic_kernel, log2n,
              dtype):
    """One radix-sort bench leg: rate, the sort's bytes-model roofline and the
    onesweep kernel's per-launch roofline."""
    return {
        "workload": workload,
        "value": round(n / (r["ms"] * 1e-3) / 1e9, 3), "unit": "Gkeys/s",
        "ms_per_step": round(r["ms"], 4), "ms_per_step_mean": round(r["ms_mean"], 4),
        "ms_per_step_min": round(r["ms_min"], 4), "ms_per_step_wall": round(r["ms_wall"], 4),
        "dtype": dtype, "bytes_model": key_bytes_model[1],
        "sort_roofline_frac": round(key_bytes_model[0] * n / (r["ms"] * 1e-3) / 1e9 /
                                    HBM_PEAK_GBS, 4),
        "roofline": roofline(pass_bytes * n, r["kernel_ms"]["radix_onesweep"], kernel_desc,
                             profiled_traffic(traffic_kernel, log2n)),
        "kernel_ms": _rounded(r["kernel_ms"]), "launches": r["launches"],
        "validated": r["validated"],
    }


def run_hbm_reference(torch, n, steps, warmup):
    """This GPU's measured HBM rates in the same run, beside the 8 TB/s peak:
    a plain device-to-device copy (torch copy_) and a read (torch sum of the
    same bytes viewed as n / 2 int64 words: torch's int32 sum widens each word
    and runs at a sixth of the read rate) of n u32 words (2^28: 1 GiB), each
    the median of event-timed steps after warm-up."""
    src = torch.ones(n, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream()

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
        for s, e in ev:
            s.record(stream)
            fn()
            e.record(stream)
        torch.cuda.synchronize()
        ms = sorted(s.elapsed_time(e) for s, e in ev)
        mid = len(ms) // 2
        return ms[mid] if len(ms) % 2 else 0.5 * (ms[mid - 1] + ms[mid])

    copy_ms = timed(lambda: dst.copy_(src))
    words = src.view(torch.int64)  # each word (1 << 32) | 1
    read_ms = timed(lambda: torch.sum(words))
    ok = bool(torch.equal(dst, src)) and \
        int(torch.sum(words).item()) == (n // 2) * ((1 << 32) + 1)
    del src, dst, words
    torch.cuda.empty_cache()
    out = {
        "workload": f"torch copy_ and sum of 2^{n.bit_length() - 1} u32 words on this GPU",
        "copy_ms": round(copy_ms, 4), "read_ms": round(read_ms, 4),
        "copy_GBps": round(8.0 * n / (copy_ms * 1e-3) / 1e9, 1),
        "read_GBps": round(4.0 * n / (read_ms * 1e-3) / 1e9, 1),
        "copy_frac_of_peak": round(8.0 * n / (copy_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "read_frac_of_peak": round(4.0 * n / (read_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
    }
    probe = _scatter_probe()
    if probe is None:
        out["scatter_probe"] = "bench_probes/libscatter_probe.so is not built"
    else:
        ok = ok and _time_scatter_probe(torch, probe, n, timed, out)
    out["validated"] = ok
    return out


def _scatter_probe():
    """bench_probes/libscatter_probe.so through ctypes, or None if not built."""
    import ctypes

    path = os.path.join(ROOT, "bench_probes", "libscatter_probe.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    lib.scatter_probe_tile_items.restype = ctypes.c_size_t
    lib.scatter_probe_tile_items.argtypes = []
    lib.scatter_probe_launch.restype = ctypes.c_int
    lib.scatter_probe_launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                         ctypes.c_int, ctypes.c_void_p]
    return lib


def _time_scatter_probe(torch, lib, n, timed, out):
    """The onesweep's memory pattern without its ranking (bench_probes/
    scatter_probe.hip): a copy through LDS, the stores of a uniform radix pass
    (256 digit runs of 68 keys per 17,408-key tile into 256 buckets), the same
    stores in 64-key-aligned windows, in two 32-lane halves per instruction, and
    with tiles placed round-robin over the XCDs, over the whole tiles of n u32 words,
    on torch's current stream. Every output is checked exactly. Adds the rates
    to `out`; returns whether every check held."""
    tile = int(lib.scatter_probe_tile_items())
    tiles = n // tile
    m = tiles * tile
    src = torch.arange(m, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream().cuda_stream

    def launch(mode):
        rc = lib.scatter_probe_launch(src.data_ptr(), dst.data_ptr(), tiles, mode, stream)
        if rc != 0:
            raise RuntimeError(f"scatter probe mode {mode}: HIP error {rc}")

    lds_copy_ms = timed(lambda: launch(0))
    ok = bool(torch.equal(dst, src))
    scatter_ms = timed(lambda: launch(1))
    want = src.view(tiles, 256, tile // 256).transpose(0, 1).contiguous().view(-1)
    ok = ok and bool(torch.equal(dst, want))
    dst.zero_()
    aligned_ms = timed(lambda: launch(2))
    ok = ok and bool(torch.equal(dst, want))
    dst.zero_()
    halves_ms = timed(lambda: launch(3))
    ok = ok and bool(torch.equal(dst, want))
    dst.zero_()
    spread_ms = timed(lambda: launch(4))
    ok = ok and bool(torch.equal(dst, want))
    del src, dst, want
    torch.cuda.empty_cache()
    moved = 8.0 * m  # bytes read + written
    out["scatter_probe"] = {
        "workload": f"{tiles} tiles of {tile} u32 keys, 512 threads x 34 keys, XCD runs of 8, "
                    "two blocks per CU (bench_probes/scatter_probe.hip)",
        "lds_copy_ms": round(lds_copy_ms, 4),
        "lds_copy_GBps": round(moved / (lds_copy_ms * 1e-3) / 1e9, 1),
        "scatter256_ms": round(scatter_ms, 4),
        "scatter256_GBps": round(moved / (scatter_ms * 1e-3) / 1e9, 1),
        "scatter256_aligned_ms": round(aligned_ms, 4),
        "scatter256_aligned_GBps": round(moved / (aligned_ms * 1e-3) / 1e9, 1),
        "scatter256_half_waves_ms": round(halves_ms, 4),
        "scatter256_half_waves_GBps": round(moved / (halves_ms * 1e-3) / 1e9, 1),
        "scatter256_no_xcd_runs_ms": round(spread_ms, 4),
        "scatter256_no_xcd_runs_GBps": round(moved / (spread_ms * 1e-3) / 1e9, 1),
        "validated": ok,
    }
    return ok


def _median_rate(fn, items, reps=5):
    """Median over `reps` runs of items / seconds of fn() (G items/s), and the
    median seconds."""
    secs = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        secs.append(time.perf_counter() - t0)
    secs.sort()
    med = secs[len(secs) // 2]
    return items / med / 1e9, med


def cpu_baseline(threads_cap=16):
    """Host baselines on this machine's cores, each the median of 5 runs over
    a bounded sample of the benchmark's own inputs (generation excluded).
    They substitute for the reference's host validation oracles and rayon
    (no Rust toolchain here): the headline is the parallel comparison sort of
    u32 keys on every core this process may use (at most 16, the GPU box's
    CPU share); beside it single-thread std::sort (slice::sort_unstable),
    std::stable_sort of u64+u32 pairs (stable sort_by_key) single- and
    multi-threaded, std::merge of u32 pairs (the reference's merge loop),
    std::set_* over u64 multisets (host_set_by) and the oracle's LSD radix
    sort."""
    import numpy as np

    import oracle
    from rccl_amd import workloads

    threads = max(1, min(threads_cap, len(os.sched_getaffinity(0))))
    out = {}
    keys26 = workloads.metric_u32_keys(1 << 26)
    v, sec = _median_rate(lambda: oracle.par_sort_unstable_u32(keys26, threads), keys26.size)
    head = {"value": round(v, 4), "unit": "Gkeys/s", "cores": threads, "kind": "port",
            "sample": f"oracle/oracle_sort.cpp parallel sort (per-thread std::sort + merge-path "
                      f"merges; substitute for rayon par_sort_unstable) of the first 2^26 keys of "
                      f"the metric input on {threads} threads, median of 5 ({sec:.3f} s each)"}
    keys22 = keys26[: 1 << 22]
    v, sec = _median_rate(lambda: oracle.sort_unstable_u32(keys22), keys22.size)
    out["u32_sort_unstable_1core"] = {
        "value": round(v, 4), "unit": "Gkeys/s", "cores": 1,
        "sample": f"std::sort (slice::sort_unstable substitute), first 2^22 metric keys, "
                  f"median of 5 ({sec:.3f} s)"}
    v, sec = _median_rate(lambda: oracle.radix_sort("u32", keys22), keys22.size)
    out["u32_lsd_radix_1core"] = {
        "value": round(v, 4), "unit": "Gkeys/s", "cores": 1,
        "sample": f"oracle/oracle.c stable LSD radix sort (8-bit passes), first 2^22 metric "
                  f"keys, median of 5 ({sec:.3f} s)"}
    del keys26
    pk, pv = workloads.metric_pairs(1 << 24)
    v, sec = _median_rate(lambda: oracle.stable_sort_pairs_u64_u32(pk, pv, threads), pk.size)
    out["pairs_par_stable_sort"] = {
        "value": round(v, 4), "unit": "Gkeys/s", "cores": threads,
        "sample": f"u64 keys + u32 values: per-thread std::stable_sort + stable merge-path "
                  f"merges (rayon par_sort substitute), first 2^24 pairs of the metric input, "
                  f"median of 5 ({sec:.3f} s)"}
    pk, pv = pk[: 1 << 22], pv[: 1 << 22]
    v, sec = _median_rate(lambda: oracle.stable_sort_pairs_u64_u32(pk, pv, 1), pk.size)
    out["pairs_stable_sort_1core"] = {
        "value": round(v, 4), "unit": "Gkeys/s", "cores": 1,
        "sample": f"std::stable_sort of u64+u32 pairs by key (stable sort_by_key substitute), "
                  f"first 2^22 metric pairs, median of 5 ({sec:.3f} s)"}
    a, pa, b, pb = workloads.c4_merge_inputs(1 << 23)
    v, sec = _median_rate(lambda: oracle.merge_pairs_u32(a, pa, b, pb), 2 * a.size)
    out["merge_1core"] = {
        "value": round(v, 4), "unit": "G outputs/s", "cores": 1,
        "sample": f"std::merge of u32 keys + u32 payloads (the reference's two-pointer merge "
                  f"substitute), C4 generator at 2^23 per side, median of 5 ({sec:.3f} s)"}
    sa, sb = workloads.c5_inputs(1 << 22)
    sets = {}
    for op in ("union", "intersection", "difference", "symmetric_difference"):
        v, sec = _median_rate(lambda op=op: oracle.std_set_op_u64(op, sa, sb), 2 * sa.size)
        sets[op] = round(v, 4)
    out["set_ops_1core"] = {
        "value": sets, "unit": "G input keys/s", "cores": 1,
        "sample": "std::set_union / set_intersection / set_difference / "
                  "set_symmetric_difference (host_set_by substitute), C5 generator at 2^22 per "
                  "side, median of 5 each"}
    head.update(out)
    return head


# ---------------------------------------------------------------------------
# C4 merge and merge sort, C5 set operations.
# ---------------------------------------------------------------------------
def run_merge(torch, np, cub, abi, DeviceBuffer, wd, log2_each, steps, warmup):
    n_each = 1 << log2_each
    a, pa, b, pb = wd.c4_merge_inputs(n_each)
    launch = cub.Program.load(0).on(torch.cuda.current_stream(0))
    A, PA, B, PB = (_buffer(torch, DeviceBuffer, t, np.uint32) for t in (a, pa, b, pb))
    out = DeviceBuffer.empty(np.uint32, 2 * n_each)
    outv = DeviceBuffer.empty(np.uint32, 2 * n_each)
    ws = cub.device_merge_pairs_workspace(launch, np.uint32, np.uint32, n_each, n_each)

    def step():
        cub.device_merge_pairs(launch, A, PA, B, PB, ws, out, outv)

    ms, ms_min, wall, kms, launches, _ = _steps(torch, abi, launch.stream(), steps, warmup, step)
    total = 2 * n_each
    ok = _sorted_equal(torch, out.tensor, torch.cat((a, b)))
    # Stability: on equal keys every A payload (high bit clear) precedes B's.
    k64 = out.tensor.to(torch.int64) & 0xFFFFFFFF
    src_b = (outv.tensor < 0)
    same = k64[1:] == k64[:-1]
    ok = ok and not bool((same & src_b[:-1] & ~src_b[1:]).any().item())
    res = {
        "workload": f"C4 DeviceMerge pairs: two sorted u32 arrays of 2^{log2_each} in [0, 2^24), "
                    "u32 payloads marking the source",
        "value": round(total / (ms * 1e-3) / 1e9, 3), "unit": "Gkeys/s (outputs)",
        "ms_per_step": round(ms, 4), "ms_per_step_wall": round(wall, 4),
        "bytes_model": "16 B/output = 8 B read (key + value) + 8 B written",
        # The whole call (partition + merge) against the same bytes.
        "leg_roofline_frac": round(16.0 * total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": roofline(16.0 * total, kms["merge"], "merge (one launch merges everything)",
                             profiled_traffic("merge", log2_each + 1)),
        "kernel_ms": _rounded(kms), "validated": bool(ok),
    }
    del a, pa, b, pb, A, PA, B, PB, out, outv, ws
    torch.cuda.empty_cache()
    return res


def run_merge_sort(torch, np, cub, abi, DeviceBuffer, wd, log2n, steps, warmup):
    n = 1 << log2n
    keys_t = wd.c4_merge_sort_keys(n)
    launch = cub.Program.load(0).on(torch.cuda.current_stream(0))
    src = _buffer(torch, DeviceBuffer, keys_t, np.uint32)
    out = DeviceBuffer.empty(np.uint32, n)
    ws = cub.device_merge_sort_workspace(launch, np.uint32, n)

    def step():
        cub.device_merge_sort_keys_copy(launch, src, ws, out)

    ms, ms_min, wall, kms, launches, per_step = _steps(torch, abi, launch.stream(), steps,
                                                           warmup, step)
    ok = _sorted_equal(torch, out.tensor, keys_t)
    res = {
        "workload": f"C4 DeviceMergeSort keys: 2^{log2n} u32 keys in [0, 2^24), ascending "
                    "(copy form: input left untouched)",
        "value": round(n / (ms * 1e-3) / 1e9, 3), "unit": "Gkeys/s",
        "ms_per_step": round(ms, 4), "ms_per_step_wall": round(wall, 4),
    }
    if "radix_onesweep" in kms:
        # Integer keys lower to the stable radix sort (same permutation), which
        # skips the passes whose byte is the same in every key (the copy form
        # runs at least one). Active passes are the bytes that vary.
        k64 = keys_t.to(torch.int64) & 0xFFFFFFFF
        active = [i for i in range(4)
                  if bool(((k64 >> (8 * i)) & 0xFF).unique().numel() > 1)] or [3]
        sweeps = [[k for name, k in st if name == "radix_onesweep"] for st in per_step]
        active_ms = [sw[i] for sw in sweeps for i in active]
        idle_ms = [sw[i] for sw in sweeps for i in range(len(sw)) if i not in active]
        key_bytes = 4 + 8 * len(active)
        res.update({
            "lowering": "stable LSD radix sort (integer keys, natural order), constant bytes "
                        "skipped",
            "radix_passes": len(active), "passes": launches.get("radix_onesweep", 0),
            "bytes_model": f"{key_bytes} B/key = 4 B (histogram) + 8 B per active radix pass",
            "roofline": roofline(8.0 * n, sum(active_ms) / len(active_ms),
                                 "radix_onesweep, active passes (one pass: 4n read + 4n write)",
                                 profiled_traffic("merge_sort_radix_onesweep", log2n + 2)),
            "idle_pass_ms": round(sum(idle_ms) / max(len(idle_ms), 1), 4),
        })
    else:
        passes = launches.get("merge_sort_pass", 0)
        key_bytes = 8 * (1 + passes)
        res.update({
            "merge_passes": passes,
            "bytes_model": f"{key_bytes} B/key = 8 B (block sort) + 8 B per merge pass",
            "roofline": roofline(8.0 * n, kms["merge_sort_pass"],
                                 "merge_sort_pass (one pass: 4n read + 4n write)",
                                 profiled_traffic("merge_sort_pass", log2n + 2)),
        })
    res.update({
        "sort_roofline_frac": round(key_bytes * n / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "kernel_ms": _rounded(kms), "validated": bool(ok),
    })
    del keys_t, src, out, ws
    torch.cuda.empty_cache()
    return res


def run_set_ops(torch, np, cub, abi, DeviceBuffer, wd, log2_each, steps, warmup):
    n_each = 1 << log2_each
    a, b = wd.c5_inputs(n_each)
    launch = cub.Program.load(0).on(torch.cuda.current_stream(0))
    A, B = (_buffer(torch, DeviceBuffer, t, np.uint64) for t in (a, b))
    out = DeviceBuffer.empty(np.uint64, 2 * n_each)
    # Reference counts from a device histogram of both multisets.
    u, inv = torch.unique(torch.cat([a, b]), return_inverse=True)
    ca = torch.bincount(inv[:n_each], minlength=u.numel())
    cb = torch.bincount(inv[n_each:], minlength=u.numel())
    want = {"union": int(torch.maximum(ca, cb).sum()), "intersection": int(torch.minimum(ca, cb).sum()),
            "difference": int((ca - cb).clamp(min=0).sum()),
            "symmetric_difference": int((ca - cb).abs().sum())}
    del u, inv, ca, cb
    results = {}
    for op in ("union", "intersection", "difference", "symmetric_difference"):
        ws = cub.device_set_workspace(launch, op, np.uint64, n_each, n_each)

        def step(op=op, ws=ws):
            cub.device_set_keys(launch, op, A, B, ws, out)

        ms, ms_min, wall, kms, _, _ = _steps(torch, abi, launch.stream(), steps, warmup, step)
        m = ws.count()
        ok = m == want[op] and _nondecreasing(torch, out.tensor[:m], 64)
        results[op] = {
            "ms_per_step": round(ms, 4), "output": m,
            "value": round(2 * n_each / (ms * 1e-3) / 1e9, 3), "unit": "Gkeys/s (inputs)",
            # The whole call (clear + partition + tile) against the tile's bytes.
            "leg_roofline_frac": round((16.0 * n_each + 8.0 * m) / (ms * 1e-3) / 1e9 /
                                       HBM_PEAK_GBS, 4),
            "roofline": roofline(16.0 * n_each + 8.0 * m, kms["set_tile"],
                                 "set_tile (reads both inputs, writes the result)",
                                 profiled_traffic("set_tile_" + op, log2_each + 2)),
            "kernel_ms": _rounded(kms), "validated": bool(ok),
        }
    del a, b, A, B, out
    torch.cuda.empty_cache()
    return {
        "workload": f"C5 set operations, keys only: sorted u64 multisets of 2^{log2_each} each "
                    "(shared pool, ~10% duplicated runs)",
        "bytes_model": "8 B read per input key + 8 B written per output key",
        **results,
    }


def run_record_sort(torch, np, abi, DeviceBuffer, wd, workloads, steps, warmup):
    """The reference's record-sort benchmark (rccl-thrust/examples/
    record_sort_benchmark.rs, benchmarks/cub-record-sort-reference.cu):
    2^20 + 13 rows of [u32; 4] with u64 payloads = row index, sorted in place
    after restoring rows and payloads from pristine device copies. As there,
    the restore copies are part of the timed step."""
    from rccl_amd import record_sort as rs
    from rccl_amd import thrust

    n, arity = workloads.RECORD_SORT_ROWS, 4
    ex = thrust.Program.load(0).par(torch.cuda.current_stream(0))
    launch = ex.launch()
    src_rows = wd.record_rows(arity, n)
    src_pay = torch.arange(n, dtype=torch.int64, device="cuda")
    rows = rs.RowBuffer(_buffer(torch, DeviceBuffer, src_rows.clone(), np.uint32), arity, n)
    pay = _buffer(torch, DeviceBuffer, src_pay.clone(), np.uint64)
    ws_bytes = abi.workspace_bytes("rccl_hip_record_sort_workspace_bytes", arity, 8, n)
    ws = DeviceBuffer.bytes(ws_bytes)
    lib = abi.load()

    def step():
        rows.words.tensor.copy_(src_rows)
        pay.tensor.copy_(src_pay)
        abi.check(lib.rccl_hip_record_sort(arity, 8, rows.ptr, pay.ptr, rows.ptr, pay.ptr, n,
                                           ws.ptr, ws_bytes, launch.handle))

    ms, ms_min, wall, kms, launches, per_step = _steps(torch, abi, launch.stream(), steps,
                                                           warmup, step)
    host_rows = workloads.record_rows(arity, n)
    order = np.lexsort(host_rows.T[::-1])  # stable: equal rows keep index order
    ok = bool(np.array_equal(rows.to_host_vec(), host_rows[order]))
    ok = ok and bool(np.array_equal(pay.to_host_vec(), order.astype(np.uint64)))
    # Byte positions in pass order (last column's low byte first) that vary
    # across the rows: the passes the library runs (an in-place sort with an
    # odd count also runs the first constant one).
    varying = [bool(np.any(((host_rows[:, arity - 1 - p // 4] >> (8 * (p % 4))) & 0xFF)
                           != ((host_rows[0, arity - 1 - p // 4] >> (8 * (p % 4))) & 0xFF)))
               for p in range(4 * arity)]
    if sum(varying) % 2:
        varying[varying.index(False)] = True
    active = [i for i, v in enumerate(varying) if v]
    sweeps = [[kms_ for name, kms_ in st if name == "record_onesweep"] for st in per_step]
    active_ms = [sw[i] for sw in sweeps for i in active]
    idle_ms = [sw[i] for sw in sweeps for i in range(len(sw)) if i not in active]
    onesweep_ms = sum(active_ms) / len(active_ms)
    sort_ms = sum(k for st in per_step for name, k in st) / len(per_step)
    res = {
        "workload": f"record sort: {n} rows of [u32; 4] (reference generator), u64 payload = "
                    "row index, in place after a device-to-device restore (both timed, as in "
                    "the reference benchmark)",
        "value": round(n / (ms * 1e-3) / 1e6, 2), "unit": "Mrows/s",
        "ms_per_step": round(ms, 4), "ms_per_step_min": round(ms_min, 4),
        "ms_per_step_wall": round(wall, 4), "sort_kernels_ms": round(sort_ms, 4),
        "active_passes": len(active), "passes": 4 * arity,
        "bytes_model": f"24 B/row moved: 48 B/row restore copies + 16 B/row histogram read + "
                       f"48 B/row per active onesweep pass ({len(active)} of {4 * arity})",
        "reference_published_ms": {"rccl_sm89": 0.437555, "cub_sm89": 0.445030,
                                   "source": "SRDATALOG_HISA_RCCL_TODO.md:180 (other hardware)"},
        "roofline": roofline(48.0 * n, onesweep_ms,
                             "record_onesweep, active passes (24 B/row read + 24 B/row write)",
                             profiled_traffic("record_onesweep_active", 28)),
        "idle_pass_ms": round(sum(idle_ms) / max(len(idle_ms), 1), 4),
        "kernel_ms": _rounded(kms), "validated": ok,
    }
    del src_rows, src_pay, rows, pay, ws
    torch.cuda.empty_cache()
    return res


def run_compaction(torch, np, abi, DeviceBuffer, workloads, steps, warmup):
    """The reference's compaction and grouped-reduction benchmarks
    (rccl-thrust/examples/compaction_benchmark.rs:62-109,
    grouped_reduction_benchmark.rs:50-80): 2^20 + 13 u32 keys = index / 3;
    unique_copy of the keys, and reduce_by_key with u64 values = index % 17 + 1
    under NaturalBagAdd."""
    n = workloads.RECORD_SORT_ROWS
    launch_stream = torch.cuda.current_stream(0)
    handle = launch_stream.cuda_stream
    idx = torch.arange(n, dtype=torch.int64, device="cuda")
    keys = _buffer(torch, DeviceBuffer, (idx // 3).to(torch.int32), np.uint32)
    vals = _buffer(torch, DeviceBuffer, idx % 17 + 1, np.uint64)
    out_k = DeviceBuffer.empty(np.uint32, n)
    out_v = DeviceBuffer.empty(np.uint64, n)
    count = DeviceBuffer.zeroed(np.uint64, 1)
    lib = abi.load()
    res = {}
    groups = (n + 2) // 3
    for name, op, pb_bytes in (("unique_copy", abi.GROUP_UNIQUE, 4.0 * n + 4.0 * groups),
                               ("reduce_by_key", abi.GROUP_OPS["natural_bag_add"],
                                12.0 * n + 12.0 * groups)):
        ws_bytes = abi.workspace_bytes("rccl_hip_group_workspace_bytes", 0, 1, op, 0, n)
        ws = DeviceBuffer.bytes(ws_bytes)

        if name == "unique_copy":
            def step(ws=ws, ws_bytes=ws_bytes):
                abi.check(lib.rccl_hip_unique_copy(0, 1, 0, keys.ptr, None, out_k.ptr, None, n,
                                                   count.ptr, ws.ptr, ws_bytes, handle))
        else:
            def step(ws=ws, ws_bytes=ws_bytes, op=op):
                abi.check(lib.rccl_hip_reduce_by_key(0, 1, op, 0, keys.ptr, None, vals.ptr,
                                                     out_k.ptr, None, out_v.ptr, n, count.ptr,
                                                     ws.ptr, ws_bytes, handle))

        ms, ms_min, wall, kms, launches, _ = _steps(torch, abi, launch_stream, steps, warmup,
                                                        step)
        c = int(count.to_host_vec()[0])
        ok = c == groups and bool(np.array_equal(out_k.to_host_vec()[:c],
                                                 np.arange(groups, dtype=np.uint32)))
        if name == "reduce_by_key":
            v = (np.arange(n) % 17 + 1).astype(np.uint64)
            expect = np.add.reduceat(v, np.arange(0, n, 3))
            ok = ok and bool(np.array_equal(out_v.to_host_vec()[:c], expect))
        res[name] = {
            "value": round(n / (ms * 1e-3) / 1e9, 3), "unit": "Gitems/s",
            "ms_per_step": round(ms, 4), "ms_per_step_min": round(ms_min, 4),
            "roofline": roofline(pb_bytes, kms["group_tile"],
                                 "group_tile (keys" + (" and values" if op else "") +
                                 " read once, one output per run)",
                                 profiled_traffic("group_tile_" + ("reduce" if op else "unique"),
                                                  28)),
            "kernel_ms": _rounded(kms), "validated": ok,
        }
    res["unique_copy"]["reference_published_ms"] = {
        "rccl_sm89": 0.018739, "cub_sm89": 0.016790,
        "source": "SRDATALOG_HISA_RCCL_TODO.md:178 (other hardware)"}
    del keys, vals, out_k, out_v, count, idx
    torch.cuda.empty_cache()
    return {
        "workload": f"{n} u32 keys = index / 3 (runs of 3); reduce_by_key values u64 = "
                    "index % 17 + 1, NaturalBagAdd",
        "bytes_model": "unique_copy 4 B/key read + 4 B/run written; reduce_by_key 12 B/item "
                       "read + 12 B/run written",
        **res,
    }


def run_search(torch, np, abi, DeviceBuffer, wd, log2_hay, log2_q, steps, warmup):
    """Vectorized lower_bound: 2^log2_hay sorted u32 keys in [0, 2^24) (the C4
    merge sort keys, sorted), 2^log2_q needles from the same distribution."""
    n, m = 1 << log2_hay, 1 << log2_q
    hay_t = torch.sort(wd.c4_merge_sort_keys(n).to(torch.int64)).values.to(torch.int32)
    q_t = wd.c4_merge_sort_keys(m)
    hay = _buffer(torch, DeviceBuffer, hay_t, np.uint32)
    q = _buffer(torch, DeviceBuffer, q_t, np.uint32)
    out = DeviceBuffer.empty(np.uint64, m)
    stream = torch.cuda.current_stream(0)
    lib = abi.load()
    ws_bytes = abi.workspace_bytes("rccl_hip_bound_search_workspace_bytes", 0, 1, n)
    ws = DeviceBuffer.bytes(ws_bytes)

    def step():
        abi.check(lib.rccl_hip_bound_search(0, 1, 0, 0, hay.ptr, n, q.ptr, m, out.ptr, ws.ptr,
                                            ws_bytes, stream.cuda_stream))

    ms, ms_min, wall, kms, launches, _ = _steps(torch, abi, stream, steps, warmup, step)
    # Validate against torch.searchsorted on the device (same definition).
    expect = torch.searchsorted(hay_t.to(torch.int64), q_t.to(torch.int64), right=False)
    ok = bool(torch.equal(out.tensor[:m], expect))
    res = {
        "workload": f"lower_bound of 2^{log2_q} u32 needles in a sorted 2^{log2_hay} u32 "
                    "haystack (values in [0, 2^24))",
        "value": round(m / (ms * 1e-3) / 1e9, 3), "unit": "Gqueries/s",
        "ms_per_step": round(ms, 4), "ms_per_step_min": round(ms_min, 4),
        "bytes_model": "12 B/query (needle read, index written); the per-call chunk index "
                       "(search_index: one read of the haystack) and the probes, one "
                       "haystack cache line per query, come on top",
        "roofline": roofline(12.0 * m, kms["search"], "search (12 B/query)",
                             profiled_traffic("search", log2_hay + 2)),
        "kernel_ms": _rounded(kms), "validated": ok,
    }
    del hay_t, q_t, hay, q, out, expect, ws
    torch.cuda.empty_cache()
    return res


def run_c1_latency(torch, np, cub, abi, DeviceBuffer, wd, steps, warmup):
    """C1 (2^20 u32 keys, cache-resident): latency of one in-place sort; and
    the single-tile route at its capacity (4,864 u32 keys: one launch)
    beside one key more (the onesweep route: init, histogram, bins scan and
    four passes)."""
    n = 1 << 20
    keys_t = wd.c1_keys(n)
    r = run_radix(torch, np, cub, abi, DeviceBuffer, keys_t, None, steps, warmup)
    small = {}
    for m in (4864, 4865):
        rs = run_radix(torch, np, cub, abi, DeviceBuffer, keys_t[:m].clone(), None, steps, warmup)
        small[str(m)] = {"us_per_sort": round(rs["ms"] * 1e3, 2), "launches": rs["launches"],
                         "validated": rs["validated"]}
    return {
        "workload": "C1 DeviceRadixSort keys-only, 2^20 u32 uniform keys, ascending "
                    "(cache-resident: latency, roofline informative only)",
        "us_per_sort": round(r["ms"] * 1e3, 2), "us_per_sort_min": round(r["ms_min"] * 1e3, 2),
        "value": round(n / (r["ms"] * 1e-3) / 1e9, 3), "unit": "Gkeys/s",
        "launches": r["launches"], "kernel_ms": _rounded(r["kernel_ms"]),
        "single_tile_route": small,
        "validated": r["validated"] and all(v["validated"] for v in small.values()),
    }


def run_reference_size(torch, np, cub, abi, DeviceBuffer, workloads, steps, warmup):
    """The workload of the reference's one published absolute radix figure: 2^24 u32 keys
    from its benchmark's xorshift fill (benchmarks/ordering-reference.cu:23-33), sorted
    ascending; 0.616 ms, 27.2 Gkeys/s on an SM89 GPU
    (reviews/current-implemented-performance.md:7,193-206). The 64 MiB keys and their
    scratch fit the MI355X's 256 MB last-level cache, so this is not an HBM-bound figure."""
    n = 1 << 24
    keys_t = torch.from_numpy(workloads.reference_bench_u32(n).view(np.int32)).to("cuda")
    r = run_radix(torch, np, cub, abi, DeviceBuffer, keys_t, None, steps, warmup)
    del keys_t
    value = n / (r["ms"] * 1e-3) / 1e9
    return {
        "workload": "DeviceRadixSort keys-only, 2^24 u32 keys from the reference benchmark's "
                    "xorshift fill, ascending, in place (cache-resident working set)",
        "value": round(value, 3), "unit": "Gkeys/s",
        "ms_per_step": round(r["ms"], 4), "ms_per_step_min": round(r["ms_min"], 4),
        "kernel_ms": _rounded(r["kernel_ms"]), "launches": r["launches"],
        "reference_published": {
            "value": 27.2, "unit": "Gkeys/s", "ms_per_step": 0.616,
            "hardware": "an NVIDIA SM89 GPU, not an MI355X",
            "source": "reviews/current-implemented-performance.md:7,193-206"},
        "ratio_to_reference_published": round(value / 27.2, 2),
        "validated": r["validated"],
    }


LEGS = ("metric", "hbm_reference", "pairs", "reference_size", "c1", "c2_uniform",
        "c2_low_entropy", "c3", "merge", "merge_sort", "set_ops", "record_sort", "compaction",
        "lower_bound", "cpu_baseline")


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=31)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--log2n", type=int, default=28)
    ap.add_argument("--legs", default=",".join(LEGS),
                    help="comma-separated legs to run (default: all): " + ", ".join(LEGS))
    ap.add_argument("--no-pairs", action="store_true", help="skip the u64+u32 pairs leg")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the reference-size, C1, C2 (uniform, low-entropy) and C3 legs")
    ap.add_argument("--no-ordering", action="store_true",
                    help="skip the C4 merge / merge sort, C5 set operation, record sort, "
                         "compaction and lower_bound legs")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--ranking", choices=("auto", "lane_atomic", "match_any"), default="auto",
                    help="onesweep ranking mode (rccl_hip_radix_configure)")
    ap.add_argument("--tile-order", choices=("auto", "ticket"), default="auto",
                    help="onesweep tile order (rccl_hip_radix_configure)")
    ap.add_argument("--calibration-copy", action="store_true",
                    help="first copy 1 GiB device to device (a kernel of known traffic for "
                         "calibrating rocprofv3's FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path).", file=sys.stderr)
        return 2
    legs = [x for x in args.legs.split(",") if x]
    unknown = sorted(set(legs) - set(LEGS))
    if unknown:
        print(f"unknown legs: {unknown}", file=sys.stderr)
        return 2
    skip = set()
    if args.no_pairs:
        skip.add("pairs")
    if args.no_configs:
        skip.update(("reference_size", "c1", "c2_uniform", "c2_low_entropy", "c3"))
    if args.no_ordering:
        skip.update(("merge", "merge_sort", "set_ops", "record_sort", "compaction",
                     "lower_bound"))
    if args.no_cpu_baseline:
        skip.add("cpu_baseline")
    legs = [x for x in legs if x not in skip]

    import numpy as np
    import torch

    from rccl_amd import _abi as abi
    from rccl_amd import cub, workloads
    from rccl_amd import workloads_device as wd
    from rccl_amd.device import DeviceBuffer

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    cub.Program.load(0)
    abi.check(abi.load().rccl_hip_radix_configure(abi.RANKING[args.ranking],
                                                  abi.TILE_ORDER[args.tile_order]))
    if args.calibration_copy:
        src = torch.empty(1 << 28, dtype=torch.int32, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    n = 1 << args.log2n
    out = {
        "metric": METRIC, "value": None, "unit": "Gkeys/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": None,
        "timing": "ms_per_step is the median of the timed steps' hipEvent intervals (the "
                  "reference's protocol); the input is restored outside each interval",
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u32",
        "data": f"synthetic: key[i] = splitmix64(0x{workloads.SEEDS['M32']:x} + i) >> 32",
        "config": {
            "workload": "DeviceRadixSort keys-only, u32 ascending, uniform 32-bit keys, "
                        f"n=2^{args.log2n}, 4 passes of 8-bit digits",
            "n": n,
            "bytes_model": "36 B/key = 4n (histogram read) + 4 x (4n read + 4n write)",
        },
        "radix_modes": {"ranking": args.ranking, "tile_order": args.tile_order},
        "legs": legs,
    }
    valid = True
    if "metric" in legs:
        _log(f"u32 keys n=2^{args.log2n}")
        keys_t = wd.metric_u32_keys(n)
        r32 = run_radix(torch, np, cub, abi, DeviceBuffer, keys_t, None, args.steps, args.warmup)
        del keys_t
        _log(f"u32 keys: {r32['ms']:.3f} ms/sort")
        out.update({
            "value": round(n / (r32["ms"] * 1e-3) / 1e9, 3),
            "ms_per_step": round(r32["ms"], 4),
            "ms_per_step_mean": round(r32["ms_mean"], 4),
            "ms_per_step_min": round(r32["ms_min"], 4),
            "ms_per_step_wall": round(r32["ms_wall"], 4),
            "sort_roofline_frac": round(36.0 * n / (r32["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "roofline": roofline(8.0 * n, r32["kernel_ms"]["radix_onesweep"],
                                 "radix_onesweep (one 8-bit pass: 4n read + 4n write)",
                                 profiled_traffic("radix_onesweep_u32", args.log2n)),
            "kernel_ms": _rounded(r32["kernel_ms"]),
            "validated": r32["validated"],
        })
        valid = valid and r32["validated"]
    if "hbm_reference" in legs:
        _log("HBM reference: device copy and read")
        ref = run_hbm_reference(torch, n, args.steps, args.warmup)
        if "metric" in legs:
            # The sort, its onesweep pass and its histogram against the rates
            # this GPU reached for a copy (read + write) and a read.
            km = out["kernel_ms"]
            ref["sort_vs_copy"] = round(36.0 * n / (out["ms_per_step"] * 1e-3) / 1e9 /
                                        ref["copy_GBps"], 4)
            ref["onesweep_vs_copy"] = round(8.0 * n / (km["radix_onesweep"] * 1e-3) / 1e9 /
                                            ref["copy_GBps"], 4)
            ref["histogram_vs_read"] = round(4.0 * n / (km["radix_histogram"] * 1e-3) / 1e9 /
                                             ref["read_GBps"], 4)
            if isinstance(ref.get("scatter_probe"), dict):
                ref["onesweep_vs_scatter256"] = round(
                    8.0 * n / (km["radix_onesweep"] * 1e-3) / 1e9 /
                    ref["scatter_probe"]["scatter256_GBps"], 4)
        out["hbm_reference"] = ref
        valid = valid and ref["validated"]
        _log(f"copy {ref['copy_GBps']} GB/s, read {ref['read_GBps']} GB/s")
        if isinstance(ref.get("scatter_probe"), dict):
            sp = ref["scatter_probe"]
            _log(f"LDS copy {sp['lds_copy_GBps']} GB/s, 256-run scatter {sp['scatter256_GBps']} GB/s")
    if "pairs" in legs:
        pk, pv = wd.metric_pairs(n)
        rp = run_radix(torch, np, cub, abi, DeviceBuffer, pk, pv, args.steps, args.warmup)
        del pk, pv
        _log(f"u64+u32 pairs: {rp['ms']:.3f} ms/sort")
        out["pairs"] = radix_leg(
            rp, n, f"DeviceRadixSort pairs, u64 keys uniform over 64 bits, u32 values = index, "
                   f"n=2^{args.log2n}, 8 passes",
            (200.0, "200 B/pair = 8n + 8 x (12n read + 12n write)"), 24.0,
            "radix_onesweep (one pass: 12n read + 12n write)", "radix_onesweep_pairs",
            args.log2n, "u64 keys + u32 values")
        valid = valid and rp["validated"]
    if "reference_size" in legs:
        _log("reference benchmark size (2^24 u32)")
        out["reference_size"] = run_reference_size(torch, np, cub, abi, DeviceBuffer, workloads,
                                                   args.steps, args.warmup)
        valid = valid and out["reference_size"]["validated"]
        _log(f"reference size: {out['reference_size']['ms_per_step']:.3f} ms")
    torch.cuda.empty_cache()
    configs = {}
    log26 = max(args.log2n - 2, 1)
    n26 = 1 << log26
    if "c1" in legs:
        _log("C1 latency")
        configs["c1"] = run_c1_latency(torch, np, cub, abi, DeviceBuffer, wd, args.steps,
                                       args.warmup)
    for name, gen, label in (("c2_uniform", wd.c2_uniform, "uniform over 64 bits"),
                             ("c2_low_entropy", wd.c2_low_entropy,
                              "256 random values, Zipf s=1.1 frequencies")):
        if name not in legs:
            continue
        _log(name)
        k, v = gen(n26)
        r = run_radix(torch, np, cub, abi, DeviceBuffer, k, v, args.steps, args.warmup)
        del k, v
        configs[name] = radix_leg(
            r, n26, f"C2 stable pair sort: 2^{log26} u64 keys ({label}), u32 values = "
                    "original index, ascending; tie order checked exactly",
            (200.0, "200 B/pair = 8n + 8 x (12n read + 12n write)"), 24.0,
            "radix_onesweep (one pass: 12n read + 12n write)", "radix_onesweep_" + name,
            args.log2n, "u64 keys + u32 values")
        _log(f"{name}: {r['ms']:.3f} ms")
    if "c3" in legs:
        _log("c3")
        k = wd.c3_keys(n).view(torch.int32)
        r = run_radix(torch, np, cub, abi, DeviceBuffer, k, None, args.steps, args.warmup,
                      kdt=np.float32, descending=True)
        del k
        configs["c3"] = radix_leg(
            r, n, f"C3 f32 keys-only descending radix sort, 2^{args.log2n} keys ~ N(0, 1e3) "
                  "with 1% +0.0, 1% -0.0, 0.1% +-inf, 0.1% denormals, 0.01% quiet NaN; bits "
                  "checked exactly (order, multiset, signed-zero tie order)",
            (36.0, "36 B/key = 4n (histogram read) + 4 x (4n read + 4n write)"), 8.0,
            "radix_onesweep (one 8-bit pass: 4n read + 4n write)", "radix_onesweep_c3",
            args.log2n, "f32 (ordered as u32 bits)")
        _log(f"c3: {r['ms']:.3f} ms")
    torch.cuda.empty_cache()
    if configs:
        out["configs"] = configs
        valid = valid and all(c["validated"] for c in configs.values())
    ordering = {}
    log_each = max(args.log2n - 1, 1)
    log_sort = max(args.log2n - 2, 1)
    if "merge" in legs:
        _log("C4 merge")
        ordering["merge"] = run_merge(torch, np, cub, abi, DeviceBuffer, wd, log_each, args.steps,
                                      args.warmup)
        _log(f"C4 merge: {ordering['merge']['ms_per_step']:.3f} ms")
    if "merge_sort" in legs:
        _log("C4 merge sort")
        ordering["merge_sort"] = run_merge_sort(torch, np, cub, abi, DeviceBuffer, wd, log_sort,
                                                args.steps, args.warmup)
        _log(f"C4 merge sort: {ordering['merge_sort']['ms_per_step']:.3f} ms")
    if "set_ops" in legs:
        _log("C5 set operations")
        ordering["set_ops"] = run_set_ops(torch, np, cub, abi, DeviceBuffer, wd, log_sort,
                                          args.steps, args.warmup)
        _log("C5 set operations done")
    if "record_sort" in legs:
        _log("record sort")
        ordering["record_sort"] = run_record_sort(torch, np, abi, DeviceBuffer, wd, workloads,
                                                  args.steps, args.warmup)
        _log(f"record sort: {ordering['record_sort']['ms_per_step']:.3f} ms")
    if "compaction" in legs:
        _log("compaction")
        ordering["compaction"] = run_compaction(torch, np, abi, DeviceBuffer, workloads,
                                                args.steps, args.warmup)
        _log("compaction done")
    if "lower_bound" in legs:
        _log("search")
        ordering["lower_bound"] = run_search(torch, np, abi, DeviceBuffer, wd, log_sort,
                                             max(log_sort - 2, 1), args.steps, args.warmup)
        _log("search done")
    if ordering:
        out["ordering"] = ordering
        for leg in ordering.values():
            if "validated" in leg:
                valid = valid and bool(leg["validated"])
            else:
                valid = valid and all(v["validated"] for v in leg.values()
                                      if isinstance(v, dict) and "validated" in v)
    if "cpu_baseline" in legs:
        _log("cpu baseline")
        out["cpu_baseline"] = cpu_baseline()
    out["validated"] = bool(valid)
    print(json.dumps(out), flush=True)
    return 0 if valid else 1


if __name__ == "__main__":
    sys.exit(main())
