import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "jero-engine_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def dev():
    """The GPU device, with the HIP library initialised on it."""
    import torch
    import jero_hip
    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a GPU")
    jero_hip.init(0)
    return torch.device("cuda", 0)
