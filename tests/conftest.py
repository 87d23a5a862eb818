"""Test configuration: the `gpu` marker, import paths and shared fixtures.

`-m "not gpu"` runs the oracle checks, host logic and C-ABI load checks on
the CPU; `-m gpu` runs the parity tests of the HIP path against the oracle.
"""
import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; parity tests of the HIP path")


def ming_pkg():
    return importlib.import_module("ming-tts-serve_amd")


@pytest.fixture(scope="session")
def ming():
    return ming_pkg()


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.lib()
    return o


@pytest.fixture(scope="session")
def ctx(ming):
    import torch

    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    c = ming.Context(0)
    yield c
    c.close()
