import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """Skip-free GPU fixture: GPU tests are selected with -m gpu and must find a GPU."""
    import torch

    assert torch.cuda.is_available(), "gpu-marked test run without a visible GPU"
    import quant_ops_amd

    assert quant_ops_amd.CUDA_AVAILABLE, f"HIP library not loaded: {quant_ops_amd._loader.LOAD_ERROR}"
    return torch.device("cuda", 0)


@pytest.fixture
def routing():
    """Switch kernel families off for one test (QO_ROUTE_* bits through the C
    ABI's qo_set_kernel_routing); the mask is cleared at teardown."""
    from quant_ops_amd import capi

    class Routing:
        def on(self, *names):
            capi.set_kernel_routing(capi.set_kernel_routing(0) | capi.route_mask(*names))

        def off(self, *names):
            capi.set_kernel_routing(capi.set_kernel_routing(0) & ~capi.route_mask(*names))

    capi.set_kernel_routing(0)
    yield Routing()
    capi.set_kernel_routing(0)
