"""The measurement probes the benchmark reports beside the decode GEMV
(runtime_amd/libminifield_probe.so): they run on the device and return
physically plausible figures.  Not part of the backend ABI."""
from __future__ import annotations

import ctypes

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu


def _probe():
    return ctypes.CDLL(str(ROOT / "runtime_amd" / "libminifield_probe.so"))


def test_shader_clock_reads_a_plausible_clock(backend):
    fn = _probe().mfp_shader_clock
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_double)]
    mhz = ctypes.c_double()
    for _ in range(2):
        assert fn(ctypes.c_void_p(backend.stream()), ctypes.byref(mhz)) == 0
        # MI355X's shader clock runs up to 2.4 GHz and does not idle below
        # a few hundred MHz while a wave executes.
        assert 300.0 < mhz.value < 3000.0, mhz.value


def test_unit_rates_are_positive_and_bounded():
    fn = _probe().mfp_unit_rates
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.POINTER(ctypes.c_double)]
    out = (ctypes.c_double * 6)()
    assert fn(out) == 0
    lds = list(out[:4])
    # LDS read rates in bytes per ns per CU: positive, and below 2 KB per
    # ns (64 banks x 4 bytes at 2.4 GHz is about 0.6 KB per ns).
    assert all(0.0 < r < 2048.0 for r in lds), lds
    # The 16-byte reads move at least as many bytes as the 4-byte ones.
    assert out[2] > out[1]
    # ns per MFMA per SIMD: 16x16x32 f16 and 16x16x64 i8 take 8 passes each.
    assert 1.0 < out[4] < 100.0 and 1.0 < out[5] < 100.0, (out[4], out[5])


def test_read_ceiling_times_a_plain_read():
    fn = _probe().mfp_read_ceiling
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_size_t, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                   ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    kb, wpb = (ctypes.c_int * 2)(1, 4), (ctypes.c_int * 2)(8, 16)
    us = (ctypes.c_double * 2)()
    nbytes = 64 << 20
    assert fn(nbytes, kb, wpb, 2, 10, us) == 0
    for t in us:
        # 64 MiB cannot stream faster than the 8 TB/s HBM peak, and a read
        # of it takes well under a millisecond.
        assert nbytes / (t * 1e-6) < 8.5e12 and t < 1000.0, t
