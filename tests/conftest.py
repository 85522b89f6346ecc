"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on CPU."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "m4-prefill-engine_amd"
for p in (ROOT, PKG, ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def oracle():
    import oracle_bindings

    oracle_bindings.lib()
    return oracle_bindings


@pytest.fixture(scope="session")
def libpath():
    import os

    p = Path(os.environ.get("M4_BRIDGE_LIB_PATH") or PKG / "libm4_bridge.so")
    if not p.exists():
        pytest.fail("libm4_bridge.so is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
    return p


@pytest.fixture(scope="session")
def bridge(libpath):
    """Initialized bridge on the GPU (gpu tests only)."""
    import m4_bridge

    b = m4_bridge.HIPBridge.get_instance(libpath)
    assert b.init(), f"m4_bridge_init failed: {b.last_error()}"
    return b
