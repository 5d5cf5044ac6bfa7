"""pytest configuration: import paths and the ``gpu`` marker.

Tests marked ``gpu`` need a ROCm device and the built libmpx_attn.so; the
rest run on CPU (oracle pins, golden fixtures, host logic, C-ABI exports).
"""

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (REPO, os.path.join(REPO, "mlx-primitives_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402  (before mlx_primitives: the HIP library binds to torch's runtime)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libmpx_attn.so")
    config.addinivalue_line("markers", "slow: full-size workloads")


@pytest.fixture(scope="session")
def device():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda:0")
