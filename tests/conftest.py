import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (test infrastructure): built on first use."""
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def rq():
    """The product package on the GPU: fails loudly if the library or device is missing."""
    import torch

    import reflex_amd

    assert torch.cuda.is_available(), "GPU test without a GPU"
    reflex_amd.init(0)
    return reflex_amd


@pytest.fixture(scope="session")
def rqh():
    """The product package for host-only calls (GGUF parsing, routing): no device needed."""
    import reflex_amd

    return reflex_amd


@pytest.fixture
def opts():
    """Setter of the library's prefill switches (rfxq_set_options) for one
    test; the previous options come back afterwards."""
    import reflex_amd

    prev = reflex_amd.get_options()
    yield lambda **changes: reflex_amd.set_options(**changes)
    reflex_amd.set_options(**prev)
