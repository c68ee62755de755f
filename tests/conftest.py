"""Shared test setup: the `gpu` marker, import paths, BF16 bit helpers.

The library times each new shape's launch candidates on first use by default (kernels/linear.py
TUNE, as engine/kernels/linear.py:494-511 does). Parity tests check particular kernels, so this
session keeps the planner's defaults unless FTK_TUNE is set; tests/test_gpu_select.py turns the
selection on itself and runs the default policy in a fresh process.
"""

import os
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "fast-transformer_amd"
for path in (str(ROOT), str(PKG)):
    if path not in sys.path:
        sys.path.insert(0, path)

GOLDEN = Path(__file__).resolve().parent / "golden"

os.environ.setdefault("FTK_TUNE", "0")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; parity tests of the HIP kernels")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def to_bits(t):
    """BF16 torch tensor (any device) -> numpy uint16 bit patterns."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def from_bits(bits, device="cpu"):
    """numpy uint16 bit patterns -> BF16 torch tensor."""
    arr = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16))
    return torch.from_numpy(arr.view(np.int16)).view(torch.bfloat16).to(device)


def seeded(shape, seed, scale=1.0, shift=0.0, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale + shift).to(torch.bfloat16).to(device)


@pytest.fixture(scope="session")
def cuda():
    return torch.device("cuda:0")
