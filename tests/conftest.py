"""Shared pytest setup: the ``gpu`` marker, repo-root import path, and GPU fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible (gpu tests run on the MI355X box)")
    from cacheir_amd import hip

    hip.load()  # raises if the HIP library was not built -- no silent fallback
    return torch.device("cuda:0")
