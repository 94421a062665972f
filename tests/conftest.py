import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_PY = os.path.join(REPO, "batmobile-evo_amd", "python")
for p in (REPO, PKG_PY):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def bm():
    """The compiled extension; fails loudly when it is not built."""
    import torch  # noqa: F401
    import _batmobile
    return _batmobile


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda:0")
