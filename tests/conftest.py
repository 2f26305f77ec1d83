"""Shared test set-up: the `gpu` marker, paths, and the built libraries."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def hip_attention():
    import torch

    import raya_amd

    if not torch.cuda.is_available():
        pytest.fail("the gpu tests need a GPU")
    return raya_amd.HipAttention()


@pytest.fixture(scope="session")
def hip_gemm():
    import torch

    import raya_amd

    if not torch.cuda.is_available():
        pytest.fail("the gpu tests need a GPU")
    return raya_amd.HipGemm()
