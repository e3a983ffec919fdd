"""Shared test setup: the `gpu` marker and import paths.

`-m "not gpu"` runs the oracle pins, the host logic and the C-ABI export
checks on a machine without a GPU; `-m gpu` runs the parity tests, which call
the HIP library through its C ABI on device 0.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "oracle", "mlx-nemo-rs_amd"):
    path = os.path.join(ROOT, sub) if sub else ROOT
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def repo_root():
    return ROOT
