"""The benchmark's device-side input generators reproduce the host
generators bit for bit when run on the GPU."""
import numpy as np
import pytest

from rccl_amd import workloads
from rccl_amd import workloads_device as wd

pytestmark = pytest.mark.gpu


def _same(t, host):
    a = t.cpu().numpy()
    return np.array_equal(a.view(np.dtype(f"u{a.dtype.itemsize}")),
                          host.view(np.dtype(f"u{host.dtype.itemsize}")))


def test_device_generators_match_host(launch):
    n = 1 << 18
    assert _same(wd.metric_u32_keys(n), workloads.metric_u32_keys(n))
    k, v = wd.metric_pairs(n)
    hk, hv = workloads.metric_pairs(n)
    assert _same(k, hk) and _same(v, hv)
    for d, h in zip(wd.c4_merge_inputs(n), workloads.c4_merge_inputs(n)):
        assert _same(d, h)
    assert _same(wd.c4_merge_sort_keys(n), workloads.c4_merge_sort_keys(n))
    for d, h in zip(wd.c5_inputs(n), workloads.c5_inputs(n)):
        assert _same(d, h)
