"""Test configuration: import paths and the `gpu` marker.

Tests marked `gpu` run the HIP kernels on a real MI355X and compare them with
the CPU oracle; everything else runs on any host (no GPU needed)."""

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
PKG_ROOT = REPO / "qvex-3.5_amd"
for p in (str(REPO), str(PKG_ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libqvex.so")


_gpu_ok = None


def gpu_available() -> bool:
    global _gpu_ok
    if _gpu_ok is None:
        import torch
        _gpu_ok = bool(torch.cuda.is_available())
    return _gpu_ok


def pytest_runtest_setup(item):
    if item.get_closest_marker("gpu") is not None and not gpu_available():
        pytest.skip("no HIP device visible")


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda:0")


def pytest_runtest_logstart(nodeid, location):
    # name the case before any GPU work starts, so a crash log points at it
    if os.environ.get("QVEX_TEST_TRACE"):
        print(f"\n[start] {nodeid}", flush=True)
