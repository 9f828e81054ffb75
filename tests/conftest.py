"""Shared pytest setup: import paths, the `gpu` marker and device helpers.

`-m "not gpu"` tests run anywhere (oracle self-checks, host logic, library
loading). `-m gpu` tests are the parity tests proper: they call the HIP
library through its C-ABI (ctypes) and compare with the CPU oracle.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("bare-metal-bard_amd", "oracle", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def gpu():
    """The CUDA(HIP) device; a GPU test on a machine without one is an error."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but torch.cuda.is_available() is False")
    import bmb
    bmb.lib()
    return torch.device("cuda:0")
