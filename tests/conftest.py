"""Test configuration: import paths, the `gpu` marker, shared helpers.

Two tiers (as in the reference's tests): CPU tests run everywhere and cover the
oracle, host-side logic and the C ABI boundary; tests marked `gpu` run the HIP
kernels on a ROCm device and compare them with the oracle.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "llm-cuda_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    from llm_cuda import _native

    _native.load()  # a missing library is an error on a GPU box, not a skip
    return torch.device("cuda", 0)
