import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "plamo-3-translate.c_amd"))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


def _build_if_missing():
    """Tests load what is built; they compile only when nothing is there."""
    if not (ROOT / "oracle" / "build" / "liboracle.so").exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True, capture_output=True)
    if not (ROOT / "plamo-3-translate.c_amd" / "libplamo_hip.so").exists():
        subprocess.run(["make", "-C", str(ROOT / "plamo-3-translate.c_amd" / "csrc")], check=True,
                       capture_output=True)


_build_if_missing()


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib
    return oracle_lib.load()


@pytest.fixture(scope="session")
def hip():
    import plamo_hip
    return plamo_hip.load()
