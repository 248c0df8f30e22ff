import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    if not os.path.exists(O.LIB_PATH):
        O.build()
    O.lib()
    return O


@pytest.fixture(scope="session")
def ctx():
    """One plugin context on device 0 for all GPU tests (fails loudly when the
    plugin or the GPU is missing: there is no fallback)."""
    import mlx_amd
    from mlx_amd import runtime
    assert mlx_amd.plugin_built(), "plugin not built: run __graft_entry__.build()"
    c = runtime.Context(0)
    yield c
    c.close()
