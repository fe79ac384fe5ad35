"""bench.py's memory-pattern probe (bench_probes/scatter_probe.hip) writes
exactly the permutation its modes describe: mode 0 copies each tile, modes 1
to 4 send run r of tile t (68 keys) to r * (tiles * 68) + t * 68. Small tile
counts, including ones that leave an XCD row of the grid partly empty."""
import ctypes
import os

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def probe():
    path = os.path.join(ROOT, "bench_probes", "libscatter_probe.so")
    lib = ctypes.CDLL(path)  # built by __graft_entry__.build(); a missing file fails here
    lib.scatter_probe_tile_items.restype = ctypes.c_size_t
    lib.scatter_probe_launch.restype = ctypes.c_int
    lib.scatter_probe_launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                         ctypes.c_int, ctypes.c_void_p]
    return lib


@pytest.mark.parametrize("tiles", [1, 7, 64, 67, 200])
def test_probe_modes_exact(launch, probe, tiles):
    import torch

    tile = int(probe.scatter_probe_tile_items())
    src = torch.arange(tiles * tile, dtype=torch.int32, device="cuda") * 7 + 3
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream().cuda_stream
    runs = src.view(tiles, 256, tile // 256).transpose(0, 1).contiguous().view(-1)
    for mode in range(5):
        dst.fill_(-1)
        assert probe.scatter_probe_launch(src.data_ptr(), dst.data_ptr(), tiles, mode,
                                          stream) == 0
        torch.cuda.synchronize()
        want = src if mode == 0 else runs
        assert torch.equal(dst, want), f"mode {mode}, {tiles} tiles"
