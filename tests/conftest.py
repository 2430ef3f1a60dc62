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


_SESSION_GRAPHS: list = []


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test without a GPU (run the CPU suite with -m 'not gpu')")
    # torch creates the CUDA generator's graph-safe state tensors when the number of live graphs goes from 0 to 1 (and
    # frees them when it drops back to 0).  Created inside torch.inference_mode -- the decoders capture their steps
    # there -- they are inference tensors, and a capture outside inference mode then fails while they live.  A small
    # graph captured here, outside inference mode and kept for the whole session, keeps the tensors normal ones, so the
    # tests' captures do not depend on the order the tests run in.
    x = torch.zeros(8, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        graph.capture_begin()
        x.add_(1)
        graph.capture_end()
    torch.cuda.current_stream().wait_stream(side)
    graph.replay()
    torch.cuda.synchronize()
    _SESSION_GRAPHS.append((graph, x))
    return torch.device("cuda")
