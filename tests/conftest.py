"""Shared test configuration: the `gpu` marker, repo paths, device helpers and error metrics."""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import aubier_amd
    aubier_amd.load_library()
    return torch.device("cuda:0")


def errs(got, ref):
    """max abs error, max abs error / max|ref|, rms error / rms(ref)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    d = np.abs(got - ref)
    mref = float(np.abs(ref).max()) or 1.0
    rms = float(np.sqrt((ref ** 2).mean())) or 1.0
    return float(d.max()), float(d.max()) / mref, float(np.sqrt((d ** 2).mean())) / rms


def say(*a):
    print(*a, flush=True)
