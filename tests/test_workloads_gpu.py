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
    assert _same(wd.c1_keys(n), workloads.c1_keys(n))
    for d, h in zip(wd.c2_uniform(n), workloads.c2_uniform(n)):
        assert _same(d, h)
    for d, h in zip(wd.c2_low_entropy(n), workloads.c2_low_entropy(n)):
        assert _same(d, h)


def test_device_c3_generator_matches_host(launch):
    """Special values and positions are bit-identical; the float64 Box-Muller
    normals may differ from the host libm's in the last place, so a normal
    value may (rarely) differ by one float32 ulp."""
    n = 1 << 18
    d = wd.c3_keys(n).cpu().numpy().view(np.uint32).astype(np.int64)
    h = workloads.c3_keys(n).view(np.uint32).astype(np.int64)
    diff = d != h
    assert int(diff.sum()) <= 4
    assert bool((np.abs(d - h) <= 1).all())
    special = ((h & 0x7FFFFFFF) == 0) | ((h & 0x7F800000) == 0x7F800000) | \
        ((h & 0x7F800000) == 0)
    assert not bool((diff & special).any())
