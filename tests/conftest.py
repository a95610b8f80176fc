"""Shared fixtures. `gpu` marks tests that need an MI355X (a HIP device)."""
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); parity tests of libfmx")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    O.build()
    return O


@pytest.fixture(scope="session")
def fmx():
    import flashmlx_amd

    flashmlx_amd.load()
    return flashmlx_amd


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device in this container")
    torch.cuda.init()
    return torch.device("cuda:0")
