import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X; the parity tests of the HIP kernels against the oracle")


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda:0")


def fp16_bits(a):
    """fp16 values as uint16 bit patterns, for bit-exact comparisons."""
    return np.ascontiguousarray(a, dtype=np.float16).view(np.uint16)
