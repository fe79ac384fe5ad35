"""GPU parity at the C4 and C5 configurations' full sizes.

C4: DeviceMerge of two sorted 2^27 u32 arrays in [0, 2^24) with source-marking
u32 payloads. C5: the four set operations, and the count-only intersection, on
two sorted 2^26 u64 multisets (shared pool, ~10% duplicated runs). Inputs come
from the device generators (bit-identical to the host generators, see
test_workloads_gpu); outputs are compared bit for bit with the oracle on host
copies of the same inputs. The C4
merge sort at full size is in test_merge_gpu.
"""
import numpy as np
import pytest

import oracle
from rccl_amd import cub
from rccl_amd import workloads_device as wd
from rccl_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu


def test_c4_merge_full_size_vs_oracle(launch):
    """2 x 2^27 sorted u32 keys with heavy duplicates; payloads are the index
    (A) or the index with the top bit set (B), so the oracle comparison also
    fixes A-before-B on ties and the order within each source."""
    a, pa, b, pb = wd.c4_merge_inputs(1 << 27)
    n_each = a.numel()
    A, PA, B, PB = (DeviceBuffer(t, np.uint32, n_each) for t in (a, pa, b, pb))
    out = DeviceBuffer.empty(np.uint32, 2 * n_each)
    outv = DeviceBuffer.empty(np.uint32, 2 * n_each)
    ws = cub.device_merge_pairs_workspace(launch, np.uint32, np.uint32, n_each, n_each)
    cub.device_merge_pairs(launch, A, PA, B, PB, ws, out, outv)
    launch.synchronize()
    got_k, got_v = out.to_host_vec(), outv.to_host_vec()
    del out, outv, ws
    host = [t.cpu().numpy().view(np.uint32) for t in (a, pa, b, pb)]
    want_k, want_v = oracle.merge("u32", host[0], host[2], host[1], host[3])
    assert np.array_equal(got_k, want_k)
    assert np.array_equal(got_v, want_v)


def test_c5_set_ops_full_size_vs_oracle(launch):
    """Union, intersection, difference and symmetric difference of the two
    2^26 u64 multisets (shared pool, ~10% duplicated runs), and the count-only
    form of intersection, against the oracle's restatement of host_set_by."""
    a, b = wd.c5_inputs(1 << 26)
    n_each = a.numel()
    A, B = DeviceBuffer(a, np.uint64, n_each), DeviceBuffer(b, np.uint64, n_each)
    ha, hb = a.cpu().numpy().view(np.uint64), b.cpu().numpy().view(np.uint64)
    out = DeviceBuffer.empty(np.uint64, 2 * n_each)
    for op in ("union", "intersection", "difference", "symmetric_difference"):
        ws = cub.device_set_workspace(launch, op, np.uint64, n_each, n_each)
        cub.device_set_keys(launch, op, A, B, ws, out)
        launch.synchronize()
        m = ws.count()
        want = oracle.set_op(op, "u64", ha, hb)
        assert m == want.size, op
        assert np.array_equal(out.to_host_vec()[:m], want), op
        if op == "intersection":
            ws2 = cub.device_set_workspace(launch, op, np.uint64, n_each, n_each)
            cub.device_set_keys(launch, op, A, B, ws2, None)
            launch.synchronize()
            assert ws2.count() == want.size
