"""Shared pytest configuration: the `gpu` marker and library builds.

CPU tests (`-m "not gpu"`) need oracle/liboracle.so; GPU tests additionally need
ornithology_amd/libornith_hip.so and a visible device. Both libraries are built
by __graft_entry__.build() (or `make -C oracle`, `make -C ornithology_amd/csrc`).
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libornith_hip.so")


@pytest.fixture(autouse=True)
def serial_prefill(monkeypatch):
    """Prompts run in the reference's ORNITH_PREFILL_SERIAL=1 mode (the token
    recurrence) unless a test sets ORNITH_PREFILL_SERIAL=0, the reference's
    default chunked delta scan."""
    monkeypatch.setenv("ORNITH_PREFILL_SERIAL", "1")


@pytest.fixture(scope="session")
def orc():
    import clibs
    return clibs.oracle()


@pytest.fixture(scope="session")
def hip_ctx():
    import ornithology_amd as oa
    ctx = oa.Context(0)
    yield ctx
    ctx.close()
