# SPDX-License-Identifier: MIT
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP engine)")


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def hip():
    """libdbs_hip through its C ABI, with torch providing device memory."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a GPU (run them with -m gpu on the GPU box)")
    from tests.hip_abi import HipEngine

    return HipEngine()
