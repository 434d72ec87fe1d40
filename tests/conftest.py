"""Test configuration: import paths, the `gpu` marker and shared helpers.

`-m "not gpu"` tests run anywhere (oracle pinning, host logic, library
exports); `-m gpu` tests need an MI355X and compare the HIP kernels, called
through libtsplat_hip.so, against the CPU oracle in oracle/.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "triposplat-cpu-avx512_amd"
ORACLE_DIR = ROOT / "oracle"
GOLDEN_DIR = ROOT / "tests" / "golden"
for p in (str(PKG_DIR), str(ORACLE_DIR), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    import oracle as O

    O.lib()
    return O


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a visible GPU")
    torch.cuda.init()
    return torch.device("cuda", 0)


@pytest.fixture(scope="session")
def hiplib(cuda):
    from tsplat import load_library

    return load_library()


def rng(seed):
    return np.random.default_rng(seed)
