"""Shared pytest setup: markers, import paths and the package handle.

The product package lives in ``continuum-attention_amd/`` (a hyphenated
directory), so it is imported with ``importlib``.
"""
import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def ca():
    return importlib.import_module("continuum-attention_amd")


@pytest.fixture(scope="session")
def gpu_ca(ca):
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a visible GPU")
    ca.native.load()  # raises loudly when the HIP library is missing
    return ca
