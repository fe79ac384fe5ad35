import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built librccl_hip.so")


def _progress(msg: str) -> None:
    # Names the case on stderr before it touches the GPU, so a run that dies
    # still says what it was doing.
    sys.stderr.write(msg + "\n")
    sys.stderr.flush()


@pytest.fixture(autouse=True)
def _announce_gpu_case(request):
    if request.node.get_closest_marker("gpu") is not None:
        _progress(f"[gpu-case] {request.node.nodeid}")
    yield


@pytest.fixture(scope="session")
def launch():
    """A CUB launch context on cuda:0's current stream."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from rccl_amd import cub

    program = cub.Program.load(0)
    return program.on(torch.cuda.current_stream(0))


@pytest.fixture(params=["default", "match_any", "ticket_tiles"])
def radix_ranking(request, launch):
    """Runs a radix test under the device's default onesweep (lane-ordered LDS
    atomics, XCD-ordered tiles on gfx950), under wave64 ballot match-any
    ranking, and with every block claiming its tile from an atomic ticket.
    The output must be identical."""
    from rccl_amd import _abi

    lib = _abi.load()
    ranking = "match_any" if request.param == "match_any" else "auto"
    order = "ticket" if request.param == "ticket_tiles" else "auto"
    _abi.check(lib.rccl_hip_radix_configure(_abi.RANKING[ranking], _abi.TILE_ORDER[order]))
    yield request.param
    _abi.check(lib.rccl_hip_radix_configure(0, 0))


@pytest.fixture(params=["auto", "ticket"])
def tile_order(request, launch):
    """Runs a look-back test (set operations, compactions) with the device's
    default tile order (XCD order on gfx950) and with every block claiming
    its tile from an atomic ticket. The output must be identical."""
    from rccl_amd import _abi

    lib = _abi.load()
    _abi.check(lib.rccl_hip_radix_configure(0, _abi.TILE_ORDER[request.param]))
    yield request.param
    _abi.check(lib.rccl_hip_radix_configure(0, 0))
