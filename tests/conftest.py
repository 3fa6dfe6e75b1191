"""Test configuration: import paths, the `gpu` marker, shared helpers.

`-m gpu` tests run the HIP kernels through the C ABI (libtrnopt_hip.so) on a ROCm GPU and compare them with
the oracle; everything else runs on the CPU (oracle pinning, host logic, the C ABI's loadable surface).
"""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "trainium-sinkhorn_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: CPU test that takes tens of seconds")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU on this machine")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def hip():
    """The HIP binding; on a GPU machine a missing library is an error, not a skip."""
    from trnopt import hip_sinkhorn as hk
    hk.lib()
    return hk


def inf_rel(a, b):
    """||a - b||_inf / ||b||_inf."""
    import numpy as np
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-300))


os.environ.setdefault("PYTHONHASHSEED", "0")
