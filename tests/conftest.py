import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "paged-infer_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")
    config.addinivalue_line("markers", "slow: long-running parity case")


def _make(path):
    # Incremental: a no-op when the library is up to date (e.g. prebuilt on the GPU box).
    subprocess.run(["make", "-s", "-C", str(path)], check=True)


@pytest.fixture(scope="session", autouse=True)
def built_libraries():
    _make(ROOT / "oracle")
    if not (ROOT / "paged-infer_amd" / "libpaged_infer_amd.so").exists():
        _make(ROOT / "paged-infer_amd")
    yield


@pytest.fixture(scope="session")
def ctx():
    import pia
    c = pia.Context(0)
    yield c
    c.close()
