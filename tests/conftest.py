"""Shared test setup: import paths, the `gpu` marker and GPU helpers."""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "rdna4-quant_amd"
for p in (ROOT, ROOT / "oracle", PKG):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built library")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device visible")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


GOLDEN = ROOT / "tests" / "golden"


def fp8_golden_table():
    """E4M3 code of every fp16 bit pattern, derived in the value domain with
    exact rationals (tests/golden/make_fp8_table.py)."""
    import numpy as np
    return np.fromfile(GOLDEN / "fp8_e4m3_from_fp16.bin", dtype=np.uint8)


def rel_l2(a, b):
    """||a - b|| / ||b|| in float64 (numpy or torch inputs)."""
    import numpy as np
    a = np.asarray(a.cpu() if hasattr(a, "cpu") else a, dtype=np.float64).ravel()
    b = np.asarray(b.cpu() if hasattr(b, "cpu") else b, dtype=np.float64).ravel()
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda:0")
