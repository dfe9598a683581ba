import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libmarlin_hip.so")


@pytest.fixture(scope="session")
def built_lib():
    """The in-tree C-ABI library; built here only when it is missing."""
    from csed499ii_amd import _lib, build

    if not _lib.LIB_PATH.exists():
        build.build()
    return _lib.load()
