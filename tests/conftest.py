import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "math-utils_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run with -m gpu on the MI355X box)")


@pytest.fixture(scope="session")
def gpu():
    """The HIP backend, required: a GPU test never passes on a CPU path."""
    import torch
    import aigpu
    aigpu.require()
    assert torch.cuda.is_available(), "torch sees no GPU"
    return aigpu
