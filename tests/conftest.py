import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "jetson-inference_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def dev():
    """The HIP device; GPU tests fail (not skip) when the library is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    import jinf_amd

    jinf_amd.lib()  # raises if libjinf_hip.so is not built
    return torch.device("cuda:0")
