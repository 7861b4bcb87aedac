"""Shared pytest configuration.

`gpu` tests need an MI355X (HIP device 0) and the built library; everything
else runs on the CPU.  The CPU suite covers the oracle against the golden
vectors, the converters, the host logic and the C-ABI exports.
"""
from __future__ import annotations

import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device and the built library")


@pytest.fixture(scope="session")
def golden_dir() -> pathlib.Path:
    return GOLDEN


@pytest.fixture(scope="session")
def backend():
    """One HipBackend on device 0 for the whole GPU session."""
    from runtime_amd.backend import HipBackend

    b = HipBackend(0)
    yield b
    b.close()


# Kernel paths of mfh_set_kernel_path: automatic (in-kernel activation
# prologue where it fits), FP32 FMA kernels only, automatic with the
# prologue as a kernel of its own.
PATHS = {"auto": 0, "fma": 1, "split": 2}


@pytest.fixture(params=list(PATHS))
def path(request, backend):
    previous = backend.set_kernel_path(PATHS[request.param])
    yield request.param
    backend.set_kernel_path(previous)


def max_rel_err(got: np.ndarray, want: np.ndarray) -> float:
    """max|got - want| / max|want| (0 when both are all-zero)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    denom = np.max(np.abs(want)) if want.size else 0.0
    diff = np.max(np.abs(got - want)) if want.size else 0.0
    return float(diff / denom) if denom > 0 else float(diff)


def assert_close(got, want, abs_tol=1e-4, rel_tol=1e-4):
    """The reference's GPU parity rule |d| <= abs + rel*|want|
    (crates/backend-wgpu/tests/parity.rs:76-87), all values finite."""
    got = np.asarray(got, dtype=np.float32)
    want = np.asarray(want, dtype=np.float32)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), "non-finite output"
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = abs_tol + rel_tol * np.abs(want.astype(np.float64))
    bad = np.argwhere(diff > bound)
    assert bad.size == 0, (
        f"{bad.shape[0]} elements exceed tolerance; first {tuple(bad[0])}: "
        f"{got[tuple(bad[0])]} vs {want[tuple(bad[0])]}")
