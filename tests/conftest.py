"""pytest configuration: import paths, the ``gpu`` marker, shared helpers."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "flaggems-sglang_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)"
    )


@pytest.fixture(scope="session")
def gpu():
    """The HIP device; GPU tests fail loudly if the library cannot load."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from flaggems_sglang import _capi

    _capi.load()
    return torch.device("cuda:0")


def pytest_sessionfinish(session, exitstatus):
    """With FGS_PARITY_LOG set, write the per-case parity figures the GPU
    tests measured (max-abs, ulps, mean_rel) to that JSON file."""
    path = os.environ.get("FGS_PARITY_LOG")
    if not path:
        return
    mod = sys.modules.get("test_fused_moe_gpu")
    rows = list(getattr(mod, "PARITY", [])) if mod else []
    import json

    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "w") as f:
        json.dump(rows, f, indent=0)
