"""Test setup: the package and the oracle importable from the repository root; the ``gpu`` marker.

``-m "not gpu"`` runs on any machine (oracle against golden vectors and closed forms, host logic, the C ABI's
exports); ``-m gpu`` runs the HIP kernels on an MI355X against the oracle.
"""

import importlib
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
importlib.import_module("omniasr-trt_amd")  # registers the package as ``omniasr_trt_amd``


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test without a GPU (run the CPU suite with -m 'not gpu')")
    return torch.device("cuda")
