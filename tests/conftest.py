"""Shared fixtures. GPU tests are marked ``gpu``: they need an MI355X and the
built libackvq.so, and fail (never skip) when either is missing."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PACKAGE_DIR = ROOT / "alelyon-compute-kit_amd"
GOLDEN = Path(__file__).resolve().parent / "golden"
for p in (str(PACKAGE_DIR), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU and the built libackvq.so")


@pytest.fixture(scope="session")
def lib():
    from alelyon_compute_kit import ack
    return ack._lib()


@pytest.fixture(scope="session")
def oracle():
    from oracle.vq4_numpy import ShaderOracle
    return ShaderOracle()


@pytest.fixture(scope="session")
def device():
    from alelyon_compute_kit import ack
    dev = ack.Device()
    yield dev
    dev.close()


@pytest.fixture(scope="session")
def vqdev(device):
    from alelyon_compute_kit import vq
    return vq.VQDevice(device)


def golden(name: str) -> dict:
    with np.load(GOLDEN / name, allow_pickle=False) as data:
        return {k: data[k] for k in data.files}
