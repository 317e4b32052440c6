"""Shared pytest configuration.

Markers:
  gpu -- needs an MI355X (gfx950) and the built libklearu_hip.so.

CPU tests (``-m "not gpu"``) pin the CPU oracle against the reference's own
known-answer tests, published vectors and closed forms, exercise host-side
logic, and check that the C-ABI library loads and exports every symbol the
header declares.  GPU tests compare the HIP path with the oracle on the same
seeded inputs.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: requires an MI355X GPU and libklearu_hip.so")


@pytest.fixture(scope="session")
def orc():
    import oracle

    return oracle


@pytest.fixture(scope="session")
def kh():
    """The product library on cuda:0 (GPU tests only)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import klearu_amd

    klearu_amd.require_gpu()
    return klearu_amd
