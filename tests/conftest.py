import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "trellis2-mojo_amd"), os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with libt2h loaded and checked to be gfx950. GPU tests fail
    (never skip) when there is no GPU or no library."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("no GPU visible: -m gpu tests need an MI355X")
    from t2h import ops

    ops.device_init(0)
    return torch.device("cuda:0")
