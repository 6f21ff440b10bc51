import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "unified-memory-scheduler_amd"
for p in (str(PKG), str(REPO / "oracle"), str(REPO)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libvbmoe.so")


@pytest.fixture(scope="session")
def vb():
    import vbmoe
    vbmoe.load()
    return vbmoe


@pytest.fixture(scope="session")
def orc():
    import oracle_py
    oracle_py.load()
    return oracle_py


@pytest.fixture(scope="session")
def gpu(vb):
    """The HIP device; a GPU test fails loudly (never falls back) if it is missing."""
    n = vb.device_count()
    assert n >= 1, "no HIP device visible"
    vb.call("vbm_set_device", 0)
    print(f"[gpu] {vb.device_name(0)}", flush=True)
    return vb
