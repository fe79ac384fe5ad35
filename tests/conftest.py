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
