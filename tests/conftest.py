"""pytest configuration: the `gpu` marker, import paths and shared fixtures.

GPU tests (`-m gpu`) call the HIP library through its C ABI and compare with
the CPU oracle (`oracle/`, test infrastructure).  CPU tests (`-m "not gpu"`)
pin the oracle itself and check the host-side logic and the library's
exported symbols without launching kernels.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

GOLDEN = ROOT / 'tests' / 'golden'


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs a ROCm GPU (MI355X) and the built HIP library')


@pytest.fixture(scope='session')
def pkg():
    return __graft_entry__.load_package()


@pytest.fixture(scope='session')
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail('GPU test collected without a visible GPU')
    return torch.device('cuda:0')
