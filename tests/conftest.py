import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "go-nngpu_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI library)")
    config.addinivalue_line("markers", "slow: full-size configuration")


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with a non-default torch stream made current, so device-API calls are
    issued on the same stream that produced their inputs; the HIP library is loaded
    and initialised (fails loudly when either is missing)."""
    import torch

    import gonngpu as G

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    torch.cuda.set_device(0)
    torch.cuda.set_stream(torch.cuda.Stream())
    G.init()
    return torch.device("cuda:0")
