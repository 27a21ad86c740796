import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    O.lib()
    O.set_threads()  # row-parallel oracle; results do not depend on the thread count
    return O


@pytest.fixture(scope="session")
def backend():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU")
    from flarellm_amd.backend import HipBackend

    b = HipBackend(0)
    print(f"[backend] {b.name()}", flush=True)
    yield b
    b.close()
