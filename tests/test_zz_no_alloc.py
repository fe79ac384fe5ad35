"""rccl_hip_radix_sort_static (no workspace argument; the control workspace
is a static device array of RCCL_HIP_STATIC_RADIX_WORKSPACE_BYTES per device)
against rccl_hip_radix_sort with a caller workspace, through the C ABI: two
calls in a row on one device, the second with a smaller input (the array
keeps the first call's contents), keys-only and pairs, both orders; outputs
bit-identical to the workspace entry point's and to the CPU oracle."""
import numpy as np
import pytest

import oracle
from rccl_amd import _abi, cub, workloads
from rccl_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu

ORDER = {False: _abi.ASCENDING, True: _abi.DESCENDING}


def _sort(launch, kind, keys, vals, descending, static):
    n = keys.size
    dk, sk = DeviceBuffer.from_host(keys), DeviceBuffer.zeroed(keys.dtype, n)
    vb = 0 if vals is None else vals.dtype.itemsize
    dv = None if vals is None else DeviceBuffer.from_host(vals)
    sv = None if vals is None else DeviceBuffer.zeroed(vals.dtype, n)
    lib = _abi.load()
    args = (_abi.KEY_KINDS[kind], vb, ORDER[descending], dk.ptr, None if dv is None else dv.ptr,
            sk.ptr, None if sv is None else sv.ptr, n)
    if static:
        _abi.check(lib.rccl_hip_radix_sort_static(*args, launch.handle))
    else:
        ws_bytes = _abi.workspace_bytes("rccl_hip_radix_sort_workspace_bytes",
                                        _abi.KEY_KINDS[kind], vb, n)
        ws = DeviceBuffer.bytes(ws_bytes)
        _abi.check(lib.rccl_hip_radix_sort(*args, ws.ptr, ws_bytes, launch.handle))
    launch.synchronize()
    return dk.to_host_vec(), (None if dv is None else dv.to_host_vec())


@pytest.mark.parametrize("descending", [False, True])
def test_static_keys_two_calls(launch, descending):
    for n in (3_000_017, 70_001):  # the second call is smaller
        keys = workloads.uniform_u32(n, 0x5A7 + n)
        keys[::7] = keys[3]  # ties
        got, _ = _sort(launch, "u32", keys, None, descending, static=True)
        ref, _ = _sort(launch, "u32", keys, None, descending, static=False)
        assert np.array_equal(got, ref)
        assert np.array_equal(got, oracle.radix_sort("u32", keys, descending=descending))


@pytest.mark.parametrize("descending", [False, True])
def test_static_pairs_two_calls(launch, descending):
    for n in (2_000_003, 40_009):
        keys, vals = workloads.c2_low_entropy(n)
        got_k, got_v = _sort(launch, "u64", keys, vals, descending, static=True)
        ref_k, ref_v = _sort(launch, "u64", keys, vals, descending, static=False)
        assert np.array_equal(got_k, ref_k) and np.array_equal(got_v, ref_v)
        want_k, want_v = oracle.radix_sort("u64", keys, vals, descending=descending)
        assert np.array_equal(got_k, want_k) and np.array_equal(got_v, want_v)


def test_static_float_descending_then_smaller(launch):
    for n in (1 << 20, 513):
        keys = workloads.c3_keys(n)
        got, _ = _sort(launch, "f32", keys, None, True, static=True)
        want = oracle.radix_sort("f32", keys, descending=True)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_static_sort_replayed_from_a_captured_graph(launch):
    """The entry point's purpose: a sort inside a captured HIP graph. After the
    program is loaded (and one eager call), the input restore and the static
    sort are captured on a side stream, then the graph is replayed four
    times with eager work (a static sort of other data, synchronizations)
    between the replays; every replay must give the oracle's output."""
    import torch

    n = 1_000_003
    keys = workloads.uniform_u32(n, 0xCA97)
    keys[::5] = keys[1]  # ties
    want = oracle.radix_sort("u32", keys)
    pristine = DeviceBuffer.from_host(keys)
    dk, sk = DeviceBuffer.zeroed(np.uint32, n), DeviceBuffer.zeroed(np.uint32, n)
    lib = _abi.load()
    kind = _abi.KEY_KINDS["u32"]
    # Eager first: the device probe and the static workspace lookup happen
    # outside the capture.
    other = workloads.uniform_u32(70_001, 0xE6E)
    got, _ = _sort(launch, "u32", other, None, False, static=True)
    assert np.array_equal(got, oracle.radix_sort("u32", other))

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=side):
        dk.tensor.copy_(pristine.tensor)
        _abi.check(lib.rccl_hip_radix_sort_static(kind, 0, _abi.ASCENDING, dk.ptr, None, sk.ptr,
                                                  None, n, torch.cuda.current_stream().cuda_stream))
    for replay in range(4):
        dk.tensor.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(dk.to_host_vec(), want), f"replay {replay}"
        got, _ = _sort(launch, "u32", other, None, replay % 2 == 1, static=True)
        assert np.array_equal(got, oracle.radix_sort("u32", other, descending=replay % 2 == 1))
