import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO, REPO / "vllm-apple_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); runs the HIP kernels")


@pytest.fixture(scope="session")
def gpu():
    """The HIP library, loaded; GPU tests fail loudly if it is missing."""
    import torch

    assert torch.cuda.is_available(), "gpu-marked test run without a ROCm device"
    from vllm_apple_amd import _lib

    lib = _lib.load()
    print(f"[gpu] {torch.cuda.get_device_name(0)} lib={_lib.library_path()}", flush=True)
    return lib
