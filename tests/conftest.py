import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    # the CPU suite must not touch the GPU: gpu tests are skipped when no
    # device is visible (they are selected explicitly with -m gpu on the box)
    import _native  # noqa: F401
    have_gpu = os.path.exists("/dev/kfd")
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU visible in this environment")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)
