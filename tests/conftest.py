import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("moss-transcribe.cpp_amd", "oracle", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _built():
    import mtg
    import oracle_py
    return os.path.exists(mtg.LIB_PATH) and os.path.exists(oracle_py.LIB_PATH)


@pytest.fixture(scope="session", autouse=True)
def _ensure_built():
    # Tests load what is built; they build only when nothing is there.
    if not _built():
        sys.path.insert(0, ROOT)
        import __graft_entry__
        __graft_entry__.build()
    yield
