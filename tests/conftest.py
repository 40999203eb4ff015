"""Shared pytest setup.

Markers: `gpu` — needs an MI355X; the parity tests proper.  Everything else
runs on the CPU (oracle pinning, host-side IR logic, library exports).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
for sub in ("wam.cpp_amd", "oracle"):
    p = str(REPO / sub)
    if p not in sys.path:
        sys.path.insert(0, p)
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); parity tests of the HIP path")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.load()
    return oracle


@pytest.fixture(scope="session")
def wx():
    import wamx
    wamx.load()
    return wamx


@pytest.fixture(scope="session")
def be(wx):
    """The HIP backend on device 0.  Fails (does not skip) without a device:
    a GPU test that cannot reach the GPU is a failure."""
    n = wx.load().wamx_get_device_count()
    if n < 1:
        pytest.fail("no HIP device visible to libwamx")
    b = wx.Backend(0)
    yield b
    b.close()


@pytest.fixture
def rng():
    return np.random.default_rng(0x5EED0000)


def rel_err(got, ref) -> float:
    """max |got - ref| / max |ref| (infinity-norm relative error)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    denom = np.max(np.abs(ref))
    return float(np.max(np.abs(got - ref)) / (denom if denom > 0 else 1.0))


def cosine(got, ref) -> float:
    a = np.asarray(got, np.float64).ravel()
    b = np.asarray(ref, np.float64).ravel()
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0 and nb == 0:
        return 1.0
    return float(a @ b / (na * nb))


# Per-op parity bar for bf16 inputs with fp32 accumulation.
REL_TOL = 1e-2
COS_TOL = 0.9999


def assert_parity(got, ref, rel=REL_TOL, cos=COS_TOL, what=""):
    r, c = rel_err(got, ref), cosine(got, ref)
    assert r <= rel and c >= cos, f"{what}: max-rel {r:.3e} (<= {rel}), cosine {c:.6f} (>= {cos})"
