"""Shared settings of the test suite: the ``gpu`` marker, and the repository root on
``sys.path`` so that ``oracle`` and ``bux_amd`` import from a checkout."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def lib():
    """The HIP library, loaded on a GPU: a GPU test fails loudly if it is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from bux_amd import _lib

    return _lib.load()
