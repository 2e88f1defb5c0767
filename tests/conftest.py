"""Shared test setup: the `gpu` marker, import paths, and GPU-test guards."""
import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO / "lemonade-burn_amd", REPO / "oracle", REPO / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")
    config.addinivalue_line("markers", "slow: long CPU oracle runs")


@pytest.fixture(scope="session")
def ctx():
    """One HIP context for the whole GPU session (one process, one stream)."""
    import lbt_hip

    c = lbt_hip.Ctx(0)
    yield c
    c.close()


def announce(msg: str):
    """Names the case on stdout before a GPU step, so a fault is attributable."""
    print(f"[gpu-case] {msg}", flush=True)
