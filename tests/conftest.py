import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "3dgs_from_scratch_amd")
for p in (ROOT, PKG, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); parity tests")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _verify_forward_orders():
    """Every blend launch order a test passes or produces is checked to permute
    each XCD tile range (cuda_rasterizer.check_forward_order)."""
    try:
        import cuda_rasterizer
    except Exception:  # the library is not built: the CPU tests do not need it
        yield
        return
    old = cuda_rasterizer.CHECK_FORWARD_ORDERS
    cuda_rasterizer.CHECK_FORWARD_ORDERS = True
    yield
    cuda_rasterizer.CHECK_FORWARD_ORDERS = old
