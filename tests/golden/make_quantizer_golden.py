"""Write tests/golden/quantizer_golden.npz from the reference quantizer.

Runs only where the reference checkout exists (this is how the committed
fixture was produced); the tests read the .npz and never import the
reference.  The quantizer is imported by file path from
  /root/reference/tools/converters/src/minifield_converters/quantization.py
(`quantize`, lines 115-160), the one function on the packed path whose
bit-exact output no reference fixture or closed form pins.

Inputs are small seeded matrices (numpy's PCG64, independent of the
backend's own generator) plus hand-built rows that sit on every rounding
boundary the algorithm has: ternary half-way quotients, INT8 half-integers,
NF4 midpoints between adjacent levels, all-zero and FP16-underflow groups,
subnormal FP16 scales and absmax values near the FP16 maximum.
"""
from __future__ import annotations

import pathlib
import sys

import numpy as np

REFERENCE_SRC = pathlib.Path("/root/reference/tools/converters/src")
OUT = pathlib.Path(__file__).resolve().parent / "quantizer_golden.npz"


def boundary_rows(scheme: str, nf4_levels: np.ndarray) -> np.ndarray:
    rows = []
    k = 256
    # A zero group followed by an FP16-underflow group.
    r = np.zeros(k, np.float32)
    r[128:] = np.float32(1e-10)
    rows.append(r)
    # Subnormal FP16 scale (absmax 3e-6) with assorted quotients.
    r = np.linspace(-3e-6, 3e-6, k).astype(np.float32)
    rows.append(r)
    # Absmax near the FP16 maximum.
    r = np.linspace(-60000.0, 65000.0, k).astype(np.float32)
    rows.append(r)
    if scheme == "ternary":
        d = np.float32(1.5)
        base = np.array([d, -d, 0.5 * d, -0.5 * d], np.float32)
        r = np.tile(base, k // 4)
        # Values one ulp either side of the half-way point.
        half = np.float32(0.5) * d
        r[4::8] = np.nextafter(half, np.float32(0))
        r[5::8] = np.nextafter(half, np.float32(10))
        r[6::8] = -np.nextafter(half, np.float32(0))
        r[7::8] = -np.nextafter(half, np.float32(10))
        rows.append(r.astype(np.float32))
    elif scheme == "int8":
        # absmax 127 -> scale 1.0 exactly: quotients are the values themselves.
        r = np.zeros(k, np.float32)
        r[0] = 127.0
        r[1:128] = (np.arange(127) - 63.0 + 0.5).astype(np.float32)
        r[128] = -127.0
        r[129:256] = np.nextafter((np.arange(127) - 63.0 + 0.5).astype(np.float32),
                                  np.float32(0))
        rows.append(r)
    else:
        # Exact midpoints between adjacent NF4 levels (ties go to the lower
        # index) and one ulp above them.
        mids = (nf4_levels[:-1] + nf4_levels[1:]) / np.float32(2)
        r = np.zeros(k, np.float32)
        r[0] = 1.0
        r[1:16] = mids
        r[16:31] = np.nextafter(mids, np.float32(2))
        r[31:46] = np.nextafter(mids, np.float32(-2))
        r[128] = -1.0
        r[129:144] = nf4_levels[:15]
        rows.append(r)
    return np.stack(rows).astype(np.float32)


def main() -> None:
    sys.path.insert(0, str(REFERENCE_SRC))
    from minifield_converters import quantization  # noqa: E402

    rng = np.random.Generator(np.random.PCG64(0x60_1DE7))
    arrays: dict[str, np.ndarray] = {}
    for scheme in ("ternary", "nf4", "int8"):
        random_rows = (rng.standard_normal((8, 256)) * 0.02).astype(np.float32)
        weights = np.concatenate([random_rows, boundary_rows(scheme, quantization.NF4)])
        codes, scales = quantization.quantize(weights, scheme)
        arrays[f"{scheme}_weights"] = weights
        arrays[f"{scheme}_codes"] = codes
        arrays[f"{scheme}_scales_f16_bits"] = scales.view(np.uint16)
        deq = quantization.dequantize(codes, scales, scheme)
        arrays[f"{scheme}_dequantized"] = deq.astype(np.float32)
    np.savez(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
