"""Shared test setup: the `gpu` marker, imports of the package and the oracle.

GPU tests call the HIP library through its C ABI (via yue2_rs_amd) and
compare against the CPU oracle (oracle/), which is test infrastructure.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


def _ensure_built():
    lib = ROOT / "yue2_rs_amd" / "lib" / "libyue2_hip.so"
    if not lib.exists():
        from yue2_rs_amd import build
        build.build()
    from oracle import oracle
    if not oracle.LIB.exists():
        oracle.build()


_ensure_built()


@pytest.fixture(scope="session")
def oracle_threads():
    from oracle import oracle
    n = int(os.environ.get("Y2_ORACLE_THREADS", min(16, os.cpu_count() or 1)))
    oracle.set_threads(n)
    return n


@pytest.fixture(scope="session")
def gpu():
    import yue2_rs_amd as y2
    if not y2.available():
        pytest.fail("no usable gfx950 device: GPU tests must not pass without one")
    return y2
