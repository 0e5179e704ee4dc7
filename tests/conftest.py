"""Test configuration: the `gpu` marker and shared helpers.

`-m "not gpu"` runs the CPU suite (oracle against golden vectors and the
compiled drinkme codec, host codec, descriptor gate, library symbols);
`-m gpu` runs the parity tests on a GPU through the C ABI.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
