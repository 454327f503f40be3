"""Test configuration: the `gpu` marker, import paths, and per-test reset of process-global state.

GPU tests (marked `gpu`) need an MI355X and the built HIP library; everything else runs on the
CPU. The repository root (for `oracle`) and torch-xdna_amd (for `torch_xdna`) go on sys.path.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "torch-xdna_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


def has_gpu():
    import torch

    return torch.cuda.is_available()


@pytest.fixture
def gpu():
    """The GPU device; fails (not skips) when a `gpu` test runs without one."""
    import torch

    assert torch.cuda.is_available(), "gpu test without a visible GPU"
    from torch_xdna import kernels

    kernels.lib()  # raises loudly if the HIP library is not built
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def reset_state():
    """Fresh process-global state per test (the reference runs each case in its own process)."""
    import torch

    yield
    from torch_xdna import conv, kernels, runtime

    runtime.stats.reset()
    runtime.decisions.clear()
    runtime._failed.clear()
    runtime._verified.clear()
    runtime._weights.clear()
    conv._layers.clear()
    kernels.reset()
    torch._dynamo.reset()
