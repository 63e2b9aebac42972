"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on the CPU."""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import voidinfer_amd  # noqa: F401  (fails loudly if the library is missing)
    assert voidinfer_amd.load().vi_init() == 0, "device is not gfx950"
    return torch.device("cuda:0")


@pytest.fixture
def rng():
    return np.random.default_rng(12345)
