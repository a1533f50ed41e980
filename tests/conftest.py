import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "bit-ttt-engine_amd")
for p in (ROOT, PKG, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture
def tune():
    """tune(name, value): set a routing / tuning knob of the library (btl_set_tuning)
    for one test; every knob touched is restored at teardown."""
    import bitlinear as bl
    saved = {}

    def set_knob(name, value):
        old = bl.set_tuning(name, int(value))
        saved.setdefault(name, old)

    yield set_knob
    for name, value in saved.items():
        bl.set_tuning(name, value)
