import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "npu-embeddings-xdna1_amd"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU")


@pytest.fixture(scope="session")
def orc():
    import orc as _orc
    return _orc.load()


@pytest.fixture(scope="session")
def ref():
    import orc as _orc
    lib = _orc.load_ref()
    if lib is None:
        pytest.skip("oracle/_ref/libref.so is not built (needs the reference checkout)")
    return lib


@pytest.fixture(scope="session")
def golden_dir():
    import pathlib
    return pathlib.Path(__file__).parent / "golden"
