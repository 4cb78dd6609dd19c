"""Shared fixtures.  `gpu` tests need an MI355X and the built library; every
other test runs on the CPU (oracle pins, ABI loading and host-only entry
points, error paths, allocator bookkeeping)."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and build/libturboquant.so")


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import load
    return load()


@pytest.fixture(scope="session")
def lib_path():
    p = ROOT / "build" / "libturboquant.so"
    if not p.exists():
        pytest.fail("build/libturboquant.so missing: run `python -m turborag_amd.build`")
    return p


@pytest.fixture(scope="session")
def tq(lib_path):
    from turborag_amd.turboquant_wrapper import TurboQuantWrapper
    return TurboQuantWrapper(lib_path)


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test on a machine without a GPU (run with -m 'not gpu')")
    return torch.device("cuda", 0)


@pytest.fixture
def rng():
    return np.random.default_rng(12345)
