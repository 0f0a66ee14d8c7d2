"""Shared fixtures. GPU tests are marked `gpu`; everything else runs on the CPU."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libgehtp.so")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def lib():
    from gehtp_amd import load_library, lib_path
    return load_library(lib_path)


@pytest.fixture(scope="session")
def engine():
    from gehtp_amd import Engine
    return Engine()


@pytest.fixture(scope="session")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


@pytest.fixture(autouse=True)
def _release_device_operands():
    yield
    import helpers
    helpers.KEEP_ALIVE.clear()
