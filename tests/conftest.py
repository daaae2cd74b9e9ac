import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for path in (ROOT, ROOT / "tsac-metal_amd", ROOT / "oracle"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def reference():
    from oracle import Reference

    if not Reference.available():
        pytest.skip("reference sources not compiled here (oracle/_ref absent)")
    return Reference()
