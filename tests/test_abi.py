"""The C-ABI library loads and exports every symbol include/*.h declares.

No compute calls: this runs without a GPU.
"""
from __future__ import annotations

import pathlib
import re
import subprocess

import pytest

from runtime_amd import _ffi

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))
DECL = re.compile(r"^\s*(?:const\s+)?[\w\s\*]*?\b(mf[hcl]_\w+)\s*\(", re.MULTILINE)


def declared_symbols() -> set[str]:
    names = set()
    for header in HEADERS:
        text = header.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.DOTALL)
        for line in text.splitlines():
            if line.strip().startswith(("typedef", "#", "}")):
                continue
            for match in DECL.finditer(line):
                names.add(match.group(1))
    return names


def exported_symbols() -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(_ffi.LIBRARY_PATH)],
                         capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.split()[-1].startswith("mf")}


def test_headers_declare_the_packed_contract():
    names = declared_symbols()
    for op in ["mfh_packed_gather_rows", "mfh_packed_linear", "mfh_packed_linear_pair",
               "mfh_packed_swiglu_linear", "mfh_packed_swiglu_pair", "mfh_fence_submit",
               "mfh_read_f32_async", "mfh_upload_u8", "mfh_upload_f32", "mfc_quantize"]:
        assert op in names


def test_library_exports_every_declared_symbol():
    missing = declared_symbols() - exported_symbols()
    assert not missing, f"declared but not exported: {sorted(missing)}"


def test_ctypes_signatures_cover_every_declaration():
    missing = declared_symbols() - set(_ffi.SIGNATURES)
    assert not missing, f"declared but without a ctypes signature: {sorted(missing)}"


def test_library_loads_and_binds():
    lib = _ffi.lib()
    for name in _ffi.SIGNATURES:
        assert getattr(lib, name) is not None
    assert lib.mfh_status_message(17) == b"backend failure"
    assert lib.mfh_status_message(9) == b"buffer belongs to another backend"


def test_library_is_built_for_gfx950():
    # The embedded offload bundle names its target triple.
    data = _ffi.LIBRARY_PATH.read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in data


def test_read_ceiling_probe_loads_and_rejects_bad_sizes():
    """The measurement probe (runtime_amd/libminifield_probe.so) exports its
    entry points and refuses arguments it cannot time before touching the
    device."""
    import ctypes
    probe = ctypes.CDLL(str(ROOT / "runtime_amd" / "libminifield_probe.so"))
    for name in ("mfp_read_ceiling", "mfp_shader_clock", "mfp_unit_rates"):
        assert hasattr(probe, name), name
    fn = probe.mfp_read_ceiling
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_size_t, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                   ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    kb, wpb, us = (ctypes.c_int * 1)(1), (ctypes.c_int * 1)(16), (ctypes.c_double * 1)()
    assert fn(1000, kb, wpb, 1, 10, us) == -1          # not a multiple of 1 KB
    assert fn(1 << 20, kb, wpb, 0, 10, us) == -1       # no launch shape
    bad_waves = (ctypes.c_int * 1)(3)
    assert fn(1 << 20, kb, bad_waves, 1, 10, us) == -1
