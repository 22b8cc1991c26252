"""Test configuration: import paths for the package (r9700-stack_amd/) and the CPU oracle (oracle/), the `gpu`
marker, and shared helpers.

`-m "not gpu"` runs the oracle's own pinning tests, the host-side layout logic and the C-ABI export check (no
kernel launches). `-m gpu` runs the parity tests proper: every HIP entry point through the C-ABI against the oracle.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "r9700-stack_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libr9k.so")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    return torch.device("cuda", 0)
