"""Shared pytest setup.

CPU tests (`-m "not gpu"`) check the oracle against closed forms, brute
force and the golden fixtures, plus the C ABI library's exports.  GPU tests
(`-m gpu`) run the HIP library through the C ABI and compare it with the
oracle on the same inputs.
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, os.path.join(REPO, "vibevoice.cpp_amd"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def vvo():
    import vvo as mod
    mod.lib()
    return mod


@pytest.fixture(scope="session")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("GPU test run without a visible GPU")
    return torch


@pytest.fixture(scope="session")
def ctx(torch_gpu):
    import vva
    c = vva.Context(0)
    yield c
    c.close()
