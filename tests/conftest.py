import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the HIP C ABI")


@pytest.fixture(autouse=True)
def _announce(request):
    # name the case before it runs, so a run that dies on the GPU still says which one
    print(f"\n[case] {request.node.nodeid}", flush=True)
    yield


@pytest.fixture(scope="session")
def backend():
    from emprise_amd import HipBackend
    b = HipBackend(0)
    yield b
    b.close()


@pytest.fixture(scope="session")
def backend_q8():
    from emprise_amd import HipBackend
    b = HipBackend(0, quantize_activations=True)
    yield b
    b.close()
