import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "lfm3-gufo-extension_amd", "python"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    # GPU tests print the case they run before touching the device.
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(pytest.mark.timeout(240))


@pytest.fixture(autouse=True)
def _announce(request):
    if "gpu" in request.keywords:
        print(f"\n[gpu case] {request.node.nodeid}", flush=True)
    yield
