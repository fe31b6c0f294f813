import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libhi2x.so")


def _have_gpu() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _have_gpu():
        return
    skip = pytest.mark.skip(reason="no HIP device in this process")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    import torch

    from hi2_amd import _lib, gptq_kernel

    d = torch.device("cuda", 0)
    # the HIP path is the product: fail loudly when it is not there
    assert _lib.load() is not None, f"libhi2x.so failed to load: {_lib.failure()}"
    assert gptq_kernel.supported(d), "not a gfx950 device"
    return d
