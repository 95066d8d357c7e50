import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP library")


def _have_gpu() -> bool:
    try:
        import rustyneedle_amd as rn
        return rn.device_count() > 0
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if any("gpu" in item.keywords for item in items) and not _have_gpu():
        skip = pytest.mark.skip(reason="no HIP device visible")
        for item in items:
            if "gpu" in item.keywords:
                item.add_marker(skip)


@pytest.fixture(scope="session")
def tiny_config():
    """A two-layer decoder with the real per-layer geometry and a small vocab."""
    import rustyneedle_amd as rn
    c = dict(rn.NEEDLE_DECODER)
    c.update(layers=2, vocab=1000, max_positions=640)
    return c


@pytest.fixture(scope="session")
def tiny_weights(tiny_config):
    import rustyneedle_amd as rn
    return rn.synthetic_weights(tiny_config, seed=7)
