"""pytest configuration: import paths and the `gpu` marker.

`-m "not gpu"` runs on a CPU-only machine: the oracle against golden vectors and
known-answer tests, host-side logic, and the C-ABI library's exports.
`-m gpu` runs the parity tests of the HIP kernels against the oracle.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "neuron-pytorch-native_amd")
KERNELS = os.path.join(PKG, "kernels")
for p in (ROOT, PKG, KERNELS, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def ops():
    """Import every op module (registers torch.ops.{deltanet,gqa,fp8,spec}.*)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import npn_ops  # noqa: F401
    return torch.ops
