"""Shared test setup: import paths and the `gpu` marker.

`-m "not gpu"` runs on any host (oracle, host logic, C-ABI exports);
`-m gpu` needs a HIP device and the built libexl3vit.so.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "exl3xpu-mixedk_amd")
for p in (ROOT, os.path.join(PKG, "quantize")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU and the built library")


def load_golden(name: str):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle as O
    O.build()
    return O


@pytest.fixture(scope="session")
def mul1_lut(oracle_mod):
    return oracle_mod.code_lut("exl3_mul1")


@pytest.fixture()
def cpu8():
    """8 torch CPU threads: the end-to-end golden vectors were written with 8,
    and CPU reductions round by their thread split."""
    import torch
    prev = torch.get_num_threads()
    torch.set_num_threads(8)
    yield
    torch.set_num_threads(prev)
