import os

# Stable CPU reduction order for the oracle's tight invariance checks (the
# reference test suite pins OMP_NUM_THREADS the same way, tests/conftest.py:5-10).
os.environ.setdefault("OMP_NUM_THREADS", "2")

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture
def gpu_device() -> torch.device:
    if not torch.cuda.is_available():
        pytest.skip("Requires a ROCm GPU")
    return torch.device("cuda")


@pytest.fixture
def bf16_autocast():
    """bf16 autocast on the GPU for the test: under it (the reference trunk's policy) fp32 inputs take the ops'
    bf16 path with fp32 in and out; outside it they take the fp32 arithmetic path."""
    with torch.autocast("cuda", dtype=torch.bfloat16):
        yield


def pytest_runtest_setup(item):
    # Name the case before any GPU work so a crash log identifies it.
    if item.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-case] {item.nodeid}", flush=True)
