"""Shared fixtures.

Markers: tests that need a GPU are marked ``gpu``; everything else runs on
the CPU (oracle vs compiled reference vs golden fixtures, host logic, and
the C-ABI library loading and exporting every declared symbol).
"""
from __future__ import annotations

import ctypes
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib
    return oracle_lib.load_oracle()


@pytest.fixture(scope="session")
def ref():
    """cogito's own sources compiled (oracle/_ref/libcgref.so)."""
    import oracle_lib
    lib = oracle_lib.load_ref()
    if lib is None:
        pytest.skip("oracle/_ref/libcgref.so not built (reference tree absent)")
    return lib


@pytest.fixture(scope="session")
def lib():
    import cogito_amd
    return cogito_amd.load()


@pytest.fixture(scope="session")
def gpu(lib):
    """The product library with an initialised device.  Fails (does not
    skip) when no HIP device is usable: GPU tests must run on the GPU."""
    rc = lib.cgx_init(0)
    if rc != 0:
        from cogito_amd.capi import last_error
        pytest.fail(f"cgx_init failed: {last_error(lib)}")
    return lib


@pytest.fixture(autouse=True)
def _fresh_error(request):
    """Each GPU test starts with an empty last-error message (the library
    keeps the last failure until it is cleared)."""
    if "gpu" in request.fixturenames:
        request.getfixturevalue("gpu").cgx_clear_error()
    yield


@pytest.fixture()
def rng():
    return np.random.default_rng(1234)
