"""Shared test setup: the `gpu` marker, import paths for the package mirror and the oracle."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "large-language-model_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs on the MI355X box)")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.lib()
    return o


@pytest.fixture(scope="session")
def mi():
    import mi_gemm

    mi_gemm.load_library()
    return mi_gemm


@pytest.fixture(scope="session")
def dev(mi):
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    mi.init()
    return torch.device("cuda:0")
