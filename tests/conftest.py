"""Shared test setup: the `gpu` marker, repo imports and the input recipe.

Inputs follow the reference tests' recipe (tests/test_flash_maxsim.py:6-9):
randn, L2-normalised per token row, cast to the kernel dtype, but drawn from a
seeded CPU generator so the oracle sees exactly the values the GPU sees.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    # GPU tests skip (not fail) on a machine without a GPU; -m "not gpu" deselects them anyway.
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def sim(shape, seed, dtype=torch.float16):
    """Reference recipe: F.normalize(randn(shape), dim=-1), cast to dtype, on CPU."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g, dtype=torch.float32)
    x = torch.nn.functional.normalize(x, dim=-1)
    return x.to(dtype)


def to_np32(t: torch.Tensor) -> np.ndarray:
    """Exact float32 values of a (CPU or GPU) fp16/bf16/fp32 tensor."""
    return t.detach().float().cpu().numpy()


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle

    if not oracle.LIB_PATH.exists():
        oracle.build()
    return oracle
