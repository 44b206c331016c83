import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "vllm-expert-pager_amd")
for p in (ROOT, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libxp.so")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(autouse=True)
def _gpu_guard(request):
    if request.node.get_closest_marker("gpu") is not None and not gpu_available():
        pytest.skip("needs a GPU")
    yield
