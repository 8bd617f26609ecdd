import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "zendnn-pytorch-plugin_amd")
for p in (ROOT, PKG_DIR, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


class _Knobs:
    """Test fixture: set library tuning knobs, restored when the test ends."""

    def __init__(self):
        self._saved = {}

    def set(self, name, value):
        import zt_capi as C
        if name not in self._saved:
            self._saved[name] = C.get_tuning(name)
        C.set_tuning(name, value)

    def restore(self):
        import zt_capi as C
        for k, v in self._saved.items():
            C.set_tuning(k, v)
        self._saved.clear()


@pytest.fixture
def knobs():
    k = _Knobs()
    yield k
    k.restore()
