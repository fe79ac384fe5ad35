#!/usr/bin/env python3
"""Benchmark of the ordering hot path on one MI355X.

Metric: Gkeys/s radix sort at 2^28 for u32 keys (the headline
``value``) and for u64-key/u32-value pairs (reported under ``pairs``), with the
fraction of the 8 TB/s HBM roofline.

A step is one full radix sort of the resident 2^28-item input. The sort is in
place, so before every step the input is restored from a pristine device copy;
that copy is outside the HIP-event interval that times the sort
(``ms_per_step``) and inside the wall-clock interval (``ms_per_step_wall``).
Per-launch kernel durations come from the library's own hipEvent timing
(rccl_hip_timing_enable), recorded on the sort's stream during the timed steps.
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


def _hash_check(torch, t):
    """Order-independent fingerprint of a device tensor: wrapping sums of the
    words and of their squares."""
    w = t.to(torch.int64)
    return int(w.sum().item()), int((w * w).sum().item())


def _sorted_unsigned(torch, t, bits):
    """True if the unsigned view of t is non-decreasing."""
    if bits == 32:
        u = t.to(torch.int64) & 0xFFFFFFFF
        return bool((u[1:] >= u[:-1]).all().item())
    # u64: compare with the sign bit flipped so signed order equals unsigned order.
    s = t ^ torch.tensor(-(1 << 63), dtype=torch.int64, device=t.device)
    return bool((s[1:] >= s[:-1]).all().item())


def run_sort(torch, cub, abi, DeviceBuffer, keys_h, values_h, steps, warmup, label):
    n = keys_h.size
    launch = cub.Program.load(0).on(torch.cuda.current_stream(0))
    stream = launch.stream()
    pristine_k = DeviceBuffer.from_host(keys_h)
    keys = DeviceBuffer.empty(keys_h.dtype, n)
    if values_h is not None:
        pristine_v = DeviceBuffer.from_host(values_h)
        values = DeviceBuffer.empty(values_h.dtype, n)
        ws = cub.device_radix_sort_pairs_workspace(launch, keys_h.dtype, values_h.dtype, n)
    else:
        ws = cub.device_radix_sort_workspace(launch, keys_h.dtype, n)

    def restore():
        keys.copy_from(pristine_k)
        if values_h is not None:
            values.copy_from(pristine_v)

    def sort():
        if values_h is not None:
            cub.device_radix_sort_pairs(launch, keys, values, ws)
        else:
            cub.device_radix_sort_keys(launch, keys, ws)

    for _ in range(warmup):
        restore()
        sort()
    torch.cuda.synchronize()

    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    abi.timing_read()
    abi.timing_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(steps):
        restore()
        starts[k].record(stream)
        sort()
        ends[k].record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    abi.timing_enable(False)
    records = abi.timing_read()
    step_ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    ms = sum(step_ms) / len(step_ms)

    kernel_ms = {}
    for name, kms, _items in records:
        kernel_ms.setdefault(name, []).append(kms)

    # Validate the last step's output: sorted, and the same multiset of keys
    # (fingerprints) and of values.
    bits = keys_h.dtype.itemsize * 8
    ok = _sorted_unsigned(torch, keys.tensor[:n] if bits == 64 else keys.tensor, bits)
    ok = ok and _hash_check(torch, keys.tensor) == _hash_check(torch, pristine_k.tensor)
    if values_h is not None:
        ok = ok and _hash_check(torch, values.tensor) == _hash_check(torch, pristine_v.tensor)
    del pristine_k, keys
    if values_h is not None:
        del pristine_v, values
    torch.cuda.empty_cache()
    return {
        "label": label,
        "n": n,
        "ms": ms,
        "ms_min": min(step_ms),
        "ms_wall": (t1 - t0) * 1e3 / steps,
        "kernel_ms": {k: sum(v) / len(v) for k, v in kernel_ms.items()},
        "kernel_launches": {k: len(v) for k, v in kernel_ms.items()},
        "validated": bool(ok),
    }


def cpu_baseline(keys_h, values_h, seconds, log2_sample):
    """Oracle LSD radix sort (single thread) on the first 2^log2_sample items
    of the same input, repeated for about `seconds`."""
    import oracle

    n = min(keys_h.size, 1 << log2_sample)
    k = keys_h[:n].copy()
    v = None if values_h is None else values_h[:n].copy()
    kind = "u32" if k.dtype.itemsize == 4 else "u64"
    reps = 0
    t0 = time.perf_counter()
    while True:
        oracle.radix_sort(kind, k, v)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    gk = reps * n / el / 1e9
    return {
        "value": round(gk, 4),
        "unit": "Gkeys/s",
        "cores": 1,
        "kind": "port",
        "sample": f"oracle/oracle.c stable LSD radix sort (8-bit passes), first 2^{log2_sample} "
                  f"{'keys' if v is None else 'pairs'} of the benchmark input, {reps} sorts in "
                  f"{el:.1f} s",
    }


def roofline(bytes_per_launch, launch_ms, traffic=None):
    achieved = bytes_per_launch / (launch_ms * 1e-3) / 1e9
    return {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--log2n", type=int, default=28)
    ap.add_argument("--no-pairs", action="store_true", help="skip the u64+u32 pairs leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path).", file=sys.stderr)
        return 2

    import torch

    from rccl_amd import _abi as abi
    from rccl_amd import cub, workloads
    from rccl_amd.device import DeviceBuffer

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    n = 1 << args.log2n
    print(f"[bench] generating inputs n=2^{args.log2n}", file=sys.stderr, flush=True)
    keys_h = workloads.metric_u32_keys(n)
    r32 = run_sort(torch, cub, abi, DeviceBuffer, keys_h, None, args.steps, args.warmup, "u32")
    print(f"[bench] u32 keys: {r32['ms']:.3f} ms/sort", file=sys.stderr, flush=True)

    rp = None
    if not args.no_pairs:
        pk, pv = workloads.metric_pairs(n)
        rp = run_sort(torch, cub, abi, DeviceBuffer, pk, pv, args.steps, args.warmup, "pairs")
        print(f"[bench] u64+u32 pairs: {rp['ms']:.3f} ms/sort", file=sys.stderr, flush=True)

    gkeys = n / (r32["ms"] * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(gkeys, 3),
        "unit": "Gkeys/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r32["ms"], 4),
        "ms_per_step_wall": round(r32["ms_wall"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": f"synthetic: key[i] = splitmix64(0x{workloads.SEEDS['M32']:x} + i) >> 32",
        "config": {
            "workload": "DeviceRadixSort keys-only, u32 ascending, uniform 32-bit keys, "
                        f"n=2^{args.log2n}, 4 passes of 8-bit digits",
            "n": n,
            "bytes_model": "36 B/key = 4n (histogram read) + 4 x (4n read + 4n write)",
        },
        "sort_roofline_frac": round(36.0 * n / (r32["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": roofline(8.0 * n, r32["kernel_ms"]["radix_onesweep"]),
        "kernel_ms": {k: round(v, 4) for k, v in r32["kernel_ms"].items()},
        "validated": r32["validated"],
    }
    out["roofline"]["kernel"] = "radix_onesweep (one 8-bit pass: 4n read + 4n write)"
    if rp is not None:
        pg = n / (rp["ms"] * 1e-3) / 1e9
        out["pairs"] = {
            "value": round(pg, 3),
            "unit": "Gkeys/s",
            "ms_per_step": round(rp["ms"], 4),
            "ms_per_step_wall": round(rp["ms_wall"], 4),
            "dtype": "u64 keys + u32 values",
            "config": {"workload": f"DeviceRadixSort pairs, u64 keys uniform over 64 bits, "
                                   f"u32 values = index, n=2^{args.log2n}, 8 passes",
                       "bytes_model": "200 B/pair = 8n + 8 x (12n read + 12n write)"},
            "sort_roofline_frac": round(200.0 * n / (rp["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "roofline": roofline(24.0 * n, rp["kernel_ms"]["radix_onesweep"]),
            "kernel_ms": {k: round(v, 4) for k, v in rp["kernel_ms"].items()},
            "validated": rp["validated"],
        }
        out["pairs"]["roofline"]["kernel"] = "radix_onesweep (one pass: 12n read + 12n write)"
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(keys_h, None, args.cpu_seconds, 24)
    print(json.dumps(out), flush=True)
    return 0 if out["validated"] and (rp is None or rp["validated"]) else 1


if __name__ == "__main__":
    sys.exit(main())
