"""Shared pytest configuration: the ``gpu`` marker and repository import path."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) GPU and the built HIP library")


def gpu_ready() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture
def cuda():
    """Device fixture for GPU tests: fails (not skips) when the HIP path cannot run."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from mingru_amd import hip_scans

    status = hip_scans.available()
    assert status is True, f"HIP backend unavailable on a GPU box: {status}"
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _no_lookback_errors(request):
    """After every GPU test: no look-back wait in this process's cached scan workspaces
    gave up (a wait that gives up leaves a partial carry, i.e. a wrong result)."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    mod = sys.modules.get("mingru_amd.hip_scans")
    if mod is None:
        return
    import torch

    if not torch.cuda.is_available():
        return
    assert mod.workspace_errors() == 0, "a look-back wait gave up during this test"
