"""GPU parity at the benchmark configurations' own shapes.

C2: stable pair sort of u64 keys with u32 values = original index, 2^26
pairs, uniform keys and low-entropy keys (256 random values with Zipf s=1.1
frequencies); the tie order must be the stable sort's. C3: f32 keys-only
descending radix sort at 2^28 with injected +0.0, -0.0, +-inf, denormals and
quiet NaNs; output bits must follow the reference's float order (BASELINE.json
configs[1] and configs[2]; rccl-cub/examples/device_radix_sort_pairs_probe.rs
:30-99, device_radix_sort_keys_probe.rs:99-246).

Two kinds of check:
- at 2^24 items, the host generators' inputs sorted on the GPU are compared
  bit for bit with the CPU oracle (oracle.radix_sort);
- at the full configuration size, the device generators' inputs (identical
  bits to the host generators, see test_workloads_gpu) are checked on the
  device for properties that together fix the output exactly: the order
  (unsigned keys non-decreasing; floats non-increasing under IEEE compare
  with the NaNs first), the same multiset of key bits, payloads that are the
  original indices of their keys, and the stable tie order (indices rising
  within each run of equal keys; the signed zeros in input order).

Every radix-sort literal vector of tests/golden also runs through the GPU.
"""
import json
import os

import numpy as np
import pytest

import oracle
from rccl_amd import cub, workloads
from rccl_amd import workloads_device as wd
from rccl_amd.device import DeviceBuffer

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("radix_ranking")]

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.json")
NP = {"u32": np.uint32, "i32": np.int32, "f32": np.float32, "u64": np.uint64,
      "i64": np.int64, "f64": np.float64}
BITS = {4: np.uint32, 8: np.uint64}


def _bits(a):
    return a.view(BITS[a.dtype.itemsize])


def _golden_radix_cases():
    with open(GOLDEN) as f:
        return [c for c in json.load(f)["cases"] if c["op"] == "radix_sort"]


def _golden_keys(case, field):
    dt = np.dtype(NP[case["kind"]])
    if case.get("float_bits"):
        return np.array([int(x, 16) for x in case[field]], dtype=BITS[dt.itemsize]).view(dt)
    return np.array(case[field], dtype=dt)


@pytest.mark.parametrize("case", _golden_radix_cases(), ids=lambda c: c["id"])
def test_golden_radix_vectors_on_gpu(launch, case):
    """The reference's literal radix vectors (signed, +-0/+-inf, the NaN bit
    order both ways, the descending signed-zero known answer), in place and
    through the DoubleBuffer form."""
    keys = _golden_keys(case, "keys")
    want = _golden_keys(case, "expected_keys")
    desc = case["descending"]
    begin, end = case.get("begin_bit", 0), case.get("end_bit", 8 * keys.dtype.itemsize)
    vals = None
    if "values" in case:
        vals = np.array(case["values"], dtype={"i32": np.int32, "u32": np.uint32,
                                               "u64": np.uint64}[case["value_dtype"]])
    k0 = DeviceBuffer.from_host(keys)
    k1 = DeviceBuffer.zeroed(keys.dtype, keys.size)
    if vals is None:
        buffers = cub.DoubleBuffer.new(k0, k1)
        ws = cub.device_radix_sort_keys_buffer_workspace(launch, keys.dtype, keys.size)
        fn = (cub.device_radix_sort_keys_buffer_descending if desc
              else cub.device_radix_sort_keys_buffer)
    else:
        v0 = DeviceBuffer.from_host(vals)
        v1 = DeviceBuffer.zeroed(vals.dtype, vals.size)
        buffers = cub.DoubleBuffer.paired((k0, v0), (k1, v1))
        ws = cub.device_radix_sort_pairs_buffer_workspace(launch, keys.dtype, vals.dtype,
                                                          keys.size)
        fn = (cub.device_radix_sort_pairs_buffer_descending if desc
              else cub.device_radix_sort_pairs_buffer)
    fn(launch, buffers, range(begin, end), ws)
    launch.synchronize()
    cur = buffers.current()
    got_k = (cur if vals is None else cur[0]).to_host_vec()
    np.testing.assert_array_equal(_bits(got_k), _bits(want))
    if vals is not None:
        np.testing.assert_array_equal(cur[1].to_host_vec(), case["expected_values"])
    # The in-place form (a full bit window only).
    if (begin, end) == (0, 8 * keys.dtype.itemsize):
        d = DeviceBuffer.from_host(keys)
        if vals is None:
            ws = cub.device_radix_sort_workspace(launch, keys.dtype, keys.size)
            (cub.device_radix_sort_keys_descending if desc else cub.device_radix_sort_keys)(
                launch, d, ws)
        else:
            dv = DeviceBuffer.from_host(vals)
            ws = cub.device_radix_sort_pairs_workspace(launch, keys.dtype, vals.dtype, keys.size)
            (cub.device_radix_sort_pairs_descending if desc else cub.device_radix_sort_pairs)(
                launch, d, dv, ws)
        launch.synchronize()
        np.testing.assert_array_equal(_bits(d.to_host_vec()), _bits(want))


# ---------------------------------------------------------------------------
# C2: u64 keys + u32 index values.
# ---------------------------------------------------------------------------
def _sort_pairs_host(launch, keys, vals):
    dk, dv = DeviceBuffer.from_host(keys), DeviceBuffer.from_host(vals)
    ws = cub.device_radix_sort_pairs_workspace(launch, np.uint64, np.uint32, keys.size)
    cub.device_radix_sort_pairs(launch, dk, dv, ws)
    launch.synchronize()
    return dk.to_host_vec(), dv.to_host_vec()


@pytest.mark.parametrize("dist", ["uniform", "low_entropy"])
def test_c2_vs_oracle_2pow24(launch, dist):
    n = 1 << 24
    keys, vals = (workloads.c2_uniform(n) if dist == "uniform"
                  else workloads.c2_low_entropy(n))
    got_k, got_v = _sort_pairs_host(launch, keys, vals)
    want_k, want_v = oracle.radix_sort("u64", keys, vals)
    assert np.array_equal(got_k, want_k)
    assert np.array_equal(got_v, want_v)
    if dist == "low_entropy":
        assert np.unique(keys).size <= 256  # the tie order was exercised


def _check_stable_pairs_device(torch, src_keys, out_keys, out_vals):
    """Exact check of a stable ascending sort of u64 keys (int64 bit patterns)
    carrying their original indices."""
    n = src_keys.numel()
    sign = torch.tensor(-(1 << 63), dtype=torch.int64, device=src_keys.device)
    u = out_keys ^ sign  # unsigned order as signed order
    assert bool((u[1:] >= u[:-1]).all()), "keys not non-decreasing"
    idx = out_vals.to(torch.int64) & 0xFFFFFFFF
    # A permutation of the indices, each value attached to its own key.
    assert bool(torch.equal(torch.sort(idx).values,
                            torch.arange(n, dtype=torch.int64, device=idx.device)))
    assert bool(torch.equal(src_keys[idx], out_keys)), "values detached from their keys"
    # Stable: indices rise within every run of equal keys.
    same = out_keys[1:] == out_keys[:-1]
    assert bool((idx[1:] > idx[:-1])[same].all()), "tie order is not the input order"
    return int(same.sum())


@pytest.mark.parametrize("dist", ["uniform", "low_entropy"])
def test_c2_full_size_device_checks(launch, dist):
    import torch

    n = 1 << 26
    keys_t, vals_t = wd.c2_uniform(n) if dist == "uniform" else wd.c2_low_entropy(n)
    dk = DeviceBuffer(keys_t.clone(), np.uint64, n)
    dv = DeviceBuffer(vals_t.clone(), np.uint32, n)
    ws = cub.device_radix_sort_pairs_workspace(launch, np.uint64, np.uint32, n)
    cub.device_radix_sort_pairs(launch, dk, dv, ws)
    launch.synchronize()
    ties = _check_stable_pairs_device(torch, keys_t, dk.tensor, dv.tensor)
    if dist == "low_entropy":
        assert ties >= n - 256  # every key but the first of its value is a tie


# ---------------------------------------------------------------------------
# C3: f32 keys-only, descending, with specials.
# ---------------------------------------------------------------------------
def test_c3_vs_oracle_2pow24(launch):
    n = 1 << 24
    keys = workloads.c3_keys(n)
    d = DeviceBuffer.from_host(keys)
    ws = cub.device_radix_sort_workspace(launch, np.float32, n)
    cub.device_radix_sort_keys_descending(launch, d, ws)
    launch.synchronize()
    got = d.to_host_vec()
    want = oracle.radix_sort("f32", keys, descending=True)
    assert np.array_equal(_bits(got), _bits(want))
    # Both signed zeros are present and appear in input order.
    zb = _bits(keys)[(_bits(keys) & np.uint32(0x7FFFFFFF)) == 0]
    assert np.array_equal(_bits(got)[(_bits(got) & np.uint32(0x7FFFFFFF)) == 0], zb)
    assert (zb == 0).any() and (zb == 0x80000000).any()


def test_c3_full_size_device_checks(launch):
    import torch

    n = 1 << 28
    keys_t = wd.c3_keys(n)
    d = DeviceBuffer(keys_t.clone().view(torch.int32), np.float32, n)
    ws = cub.device_radix_sort_workspace(launch, np.float32, n)
    cub.device_radix_sort_keys_descending(launch, d, ws)
    launch.synchronize()
    out_bits = d.tensor
    src_bits = keys_t.view(torch.int32)
    counts = workloads.c3_special_counts(n)
    # The same multiset of bit patterns.
    assert bool(torch.equal(torch.sort(out_bits).values, torch.sort(src_bits).values))
    out = out_bits.view(torch.float32)
    # All NaNs (one positive quiet pattern) come first in descending order.
    k = counts["nan"]
    assert bool(torch.isnan(out[:k]).all()) and not bool(torch.isnan(out[k:]).any())
    # The rest is non-increasing under IEEE compare (-0.0 == +0.0).
    rest = out[k:]
    assert bool((rest[1:] <= rest[:-1]).all()), "not descending"
    # The signed zeros form one run holding them in input order.
    zmask_out = (out_bits & 0x7FFFFFFF) == 0
    zmask_src = (src_bits & 0x7FFFFFFF) == 0
    assert int(zmask_out.sum()) == counts["+0"] + counts["-0"]
    assert bool(torch.equal(out_bits[zmask_out], src_bits[zmask_src])), "signed-zero tie order"
    # Infinities at the ends of the numbers, denormals around the zeros.
    assert bool(torch.isposinf(rest[:counts["+inf"]]).all())
    assert bool(torch.isneginf(rest[rest.numel() - counts["-inf"]:]).all())



# ---------------------------------------------------------------------------
# The metric's own shapes (bench.py's headline and pairs legs).
# ---------------------------------------------------------------------------
def test_metric_u32_keys_full_size(launch):
    """2^28 u32 keys ascending from bench.py's device generator: the output
    equals the input sorted by torch.sort (unsigned order through a flipped
    sign bit), word for word."""
    import torch

    n = 1 << 28
    keys_t = wd.metric_u32_keys(n)
    d = DeviceBuffer(keys_t.clone(), np.uint32, n)
    ws = cub.device_radix_sort_workspace(launch, np.uint32, n)
    cub.device_radix_sort_keys(launch, d, ws)
    launch.synchronize()
    sign = torch.tensor(-(1 << 31), dtype=torch.int32, device=keys_t.device)
    want = torch.sort(keys_t ^ sign).values ^ sign
    del keys_t
    assert bool(torch.equal(d.tensor, want))


def test_metric_pairs_full_size(launch):
    """2^28 u64 keys with u32 values = original index, ascending, from
    bench.py's device generator: keys non-decreasing, every value the index
    of its own key, indices a permutation and rising within runs of equal
    keys; together these fix the stable sort's output exactly."""
    import torch

    n = 1 << 28
    keys_t, vals_t = wd.metric_pairs(n)
    dk = DeviceBuffer(keys_t.clone(), np.uint64, n)
    dv = DeviceBuffer(vals_t.clone(), np.uint32, n)
    del vals_t
    ws = cub.device_radix_sort_pairs_workspace(launch, np.uint64, np.uint32, n)
    cub.device_radix_sort_pairs(launch, dk, dv, ws)
    launch.synchronize()
    _check_stable_pairs_device(torch, keys_t, dk.tensor, dv.tensor)
