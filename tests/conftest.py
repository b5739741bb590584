"""Shared pytest setup: the `gpu` marker, the repository on sys.path, and the
CPU oracle built on first use."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built liblrmoe.so")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    if not O.LIB.exists():
        O.build(ref=False)
    return O


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from lightreason_amd import _native

    _native.device_check()
    return torch.device("cuda:0")


SEED = 4242


@pytest.fixture(scope="session")
def model(device):
    """One synthetic layer (256 resident experts, router, shared expert,
    RMSNorm weight) shared by the GPU test modules."""
    from lightreason_amd.synthetic import SyntheticModel

    return SyntheticModel(layers=1, device=device, seed=SEED, shared=True, norm="normal")


@pytest.fixture(scope="session")
def host_experts(model):
    from helpers import HostExperts

    return HostExperts(model.bank, 0)
