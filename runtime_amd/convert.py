"""numpy front end of the converters in include/minifield_convert.h:
the group-128 quantizer (a restatement of
tools/converters/src/minifield_converters/quantization.py:115-160) and the
seeded synthetic-input generator used for workloads."""
from __future__ import annotations

import os

import numpy as np

from . import _ffi

FORMATS = {"ternary": 0, "nf4": 1, "int8": 2}
BITS = {"ternary": 2, "nf4": 4, "int8": 8}


class ConversionError(ValueError):
    """Rejected quantizer input (quantization.py raises ConversionError)."""


def _threads(threads: int | None) -> int:
    return threads if threads is not None else min(16, os.cpu_count() or 1)


def quantize(weights: np.ndarray, scheme: str, threads: int | None = None):
    """Return (codes u8 [rows, k*bits/8], scales f16 [rows, k/128])."""
    w = np.ascontiguousarray(weights, dtype=np.float32)
    if w.ndim != 2:
        raise ConversionError("weights must be a non-empty real numeric matrix")
    rows, k = w.shape
    if scheme not in FORMATS:
        raise ConversionError("quantization scheme must be ternary, nf4, or int8")
    width = k * BITS[scheme] // 8 if k % 128 == 0 else 0
    codes = np.empty((rows, width), dtype=np.uint8)
    scales = np.empty((rows, k // 128 if k % 128 == 0 else 0), dtype=np.uint16)
    status = _ffi.lib().mfc_quantize(
        w.ctypes.data_as(_ffi.c_float_p), rows, k, FORMATS[scheme],
        codes.ctypes.data_as(_ffi.c_u8_p), scales.ctypes.data_as(_ffi.c_u16_p),
        _threads(threads))
    if status:
        raise ConversionError("weights must be finite FP32 rows with K%128=0 and FP16 scales")
    return codes, scales.view(np.float16)


def dequantize(codes: np.ndarray, scales: np.ndarray, scheme: str) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    s = np.ascontiguousarray(scales, dtype=np.float16).view(np.uint16)
    rows = c.shape[0]
    k = c.shape[1] * 8 // BITS[scheme]
    out = np.empty((rows, k), dtype=np.float32)
    status = _ffi.lib().mfc_dequantize(c.ctypes.data_as(_ffi.c_u8_p),
                                       s.ctypes.data_as(_ffi.c_u16_p), rows, k,
                                       FORMATS[scheme], out.ctypes.data_as(_ffi.c_float_p))
    if status:
        raise ConversionError("packed codes hold a reserved value")
    return out


def f16_to_f32(scales: np.ndarray) -> np.ndarray:
    """The loader's F16 -> F32 scale decode (executor-core/src/loader.rs:408-421)."""
    s = np.ascontiguousarray(scales, dtype=np.float16).view(np.uint16)
    out = np.empty(s.shape, dtype=np.float32)
    _ffi.lib().mfc_f16_to_f32_array(s.ctypes.data_as(_ffi.c_u16_p),
                                    out.ctypes.data_as(_ffi.c_float_p), s.size)
    return out


def normal(shape, seed: int, sigma: float = 1.0, mean: float = 0.0,
           threads: int | None = None) -> np.ndarray:
    """Seeded N(mean, sigma) f32 samples (splitmix64 + Box-Muller in f64)."""
    out = np.empty(int(np.prod(shape)), dtype=np.float32)
    _ffi.lib().mfc_fill_normal(out.ctypes.data_as(_ffi.c_float_p), out.size,
                               seed & 0xFFFFFFFFFFFFFFFF, mean, sigma, _threads(threads))
    return out.reshape(shape)


def token_ids(count: int, seed: int, vocab: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint32)
    _ffi.lib().mfc_fill_token_ids(out.ctypes.data_as(_ffi.c_u32_p), count, seed, vocab)
    return out


def packed_weights(rows: int, k: int, scheme: str, seed: int, sigma: float = 0.02,
                   threads: int | None = None):
    """Seeded N(0, sigma) dense weights quantized to (codes, f16 scales)."""
    dense = normal((rows, k), seed, sigma, threads=threads)
    return quantize(dense, scheme, threads=threads)
