import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "conflux-nova_amd", ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu on the GPU box)")


@pytest.fixture(scope="session")
def oracle():
    from oracle_py import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def reference():
    """The reference's own code built into oracle/_ref (None where the
    reference tree was absent at build time, e.g. on the GPU box)."""
    from oracle_py import Reference
    return Reference() if Reference.available() else None


def nova_lib(model):
    import nova_amd
    return nova_amd.load(model)


@pytest.fixture(scope="session")
def nova7():
    return nova_lib("qwen25_7b")


@pytest.fixture(scope="session")
def nova15():
    return nova_lib("qwen25_1p5b")


@pytest.fixture(scope="session")
def nova14():
    return nova_lib("qwen25_14b")
