"""GPU parity for radix sorts of 2^30 items and more.

From 2^30 items the onesweep's look-back descriptors are 64-bit: a digit's
prefix count can then reach 2^30, which no longer fits beside the two flag
bits of a 32-bit descriptor (rccl_amd/csrc/radix.hip, layout). The reference
sorts such inputs with the same stable LSD passes
(rccl-cub/examples/device_radix_sort_pairs_probe.rs:30-99 checks the stable
pair order these tests check).

n = 2^30 + 4099 (a partial last tile). The keys are narrower than their type,
so in the top pass(es) every item has the same digit and that digit's prefix
counts pass 2^30; each key value recurs about 64 times (u32) or is nearly
unique (u64). The values are the original indices. Checked on the device,
with the same force as a comparison with the oracle: the keys are
non-decreasing, the values are a permutation of the indices, each value sits
beside its own key, and indices rise within every run of equal keys. Only a
stable sort satisfies all four, and it is unique.
"""
import numpy as np
import pytest

from rccl_amd import cub
from rccl_amd import workloads_device as wd
from rccl_amd.device import DeviceBuffer

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("radix_ranking")]

N = (1 << 30) + 4099
SEED = 0x5EED_0030


def _check_stable_index_pairs(torch, src_keys, out_keys, out_vals):
    """Exact check of a stable ascending sort of non-negative keys carrying
    their original indices."""
    n = src_keys.numel()
    assert bool((out_keys[1:] >= out_keys[:-1]).all()), "keys not non-decreasing"
    idx = out_vals.to(torch.int64)
    assert int(idx.min()) >= 0 and int(idx.max()) < n
    assert bool((torch.bincount(idx, minlength=n) == 1).all()), "values not a permutation"
    assert bool(torch.equal(src_keys[idx], out_keys)), "values detached from their keys"
    same = out_keys[1:] == out_keys[:-1]
    assert bool((idx[1:] > idx[:-1])[same].all()), "tie order is not the input order"
    return int(same.sum())


def test_u32_pairs_wide(launch):
    """24-bit u32 keys with u32 indices: the top pass has one digit for all
    items."""
    import torch

    keys = wd.shr(wd.hash_range(SEED, N), 40).to(torch.int32)
    vals = torch.arange(N, dtype=torch.int32, device=keys.device)
    dk = DeviceBuffer(keys.clone(), np.uint32, N)
    dv = DeviceBuffer(vals, np.uint32, N)
    ws = cub.device_radix_sort_pairs_workspace(launch, np.uint32, np.uint32, N)
    cub.device_radix_sort_pairs(launch, dk, dv, ws)
    launch.synchronize()
    del ws
    ties = _check_stable_index_pairs(torch, keys, dk.tensor, dv.tensor)
    assert ties >= N - (1 << 24)  # at most 2^24 distinct keys


def test_u64_pairs_wide(launch):
    """40-bit u64 keys with u64 indices: the top three passes have one digit
    for all items."""
    import torch

    keys = wd.shr(wd.hash_range(SEED + 1, N), 24)
    vals = torch.arange(N, dtype=torch.int64, device=keys.device)
    dk = DeviceBuffer(keys.clone(), np.uint64, N)
    dv = DeviceBuffer(vals, np.uint64, N)
    ws = cub.device_radix_sort_pairs_workspace(launch, np.uint64, np.uint64, N)
    cub.device_radix_sort_pairs(launch, dk, dv, ws)
    launch.synchronize()
    del ws
    _check_stable_index_pairs(torch, keys, dk.tensor, dv.tensor)


def test_u32_keys_wide_descending(launch):
    """Full-width u32 keys, keys only, descending: the same multiset of key
    bits in non-increasing unsigned order."""
    import torch

    keys = wd.shr(wd.hash_range(SEED + 2, N), 32).to(torch.int32)
    d = DeviceBuffer(keys.clone(), np.uint32, N)
    ws = cub.device_radix_sort_workspace(launch, np.uint32, N)
    cub.device_radix_sort_keys_descending(launch, d, ws)
    launch.synchronize()
    del ws
    sign = torch.tensor(-(1 << 31), dtype=torch.int32, device=keys.device)
    got = d.tensor ^ sign  # unsigned order as signed order
    assert bool((got[1:] <= got[:-1]).all()), "keys not non-increasing"
    want = torch.sort(keys ^ sign, descending=True).values
    assert bool(torch.equal(got, want)), "not the same multiset of keys"
