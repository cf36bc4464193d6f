import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def device():
    import torch

    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _announce_gpu_test(request):
    """Name every GPU test on the real stderr before it runs, so a run that dies mid-test
    still says which case it was in."""
    if "gpu" in request.keywords:
        sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
        sys.__stderr__.flush()
    yield
