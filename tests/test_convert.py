"""The backend's converters against the reference quantizer.

`quantizer_golden.npz` holds outputs of the reference's
tools/converters/src/minifield_converters/quantization.py:quantize on seeded
and boundary matrices (written by tests/golden/make_quantizer_golden.py);
the hand-computed bytes come from tools/converters/tests/test_quantization.py.
"""
from __future__ import annotations

import numpy as np
import pytest

from runtime_amd import convert

SCHEMES = ["ternary", "nf4", "int8"]


@pytest.fixture(scope="module")
def golden(golden_dir):
    return np.load(golden_dir / "quantizer_golden.npz")


@pytest.mark.parametrize("scheme", SCHEMES)
def test_quantize_matches_reference_golden_bitwise(golden, scheme):
    codes, scales = convert.quantize(golden[f"{scheme}_weights"], scheme)
    assert codes.tobytes() == golden[f"{scheme}_codes"].tobytes()
    assert scales.view(np.uint16).tobytes() == golden[f"{scheme}_scales_f16_bits"].tobytes()


@pytest.mark.parametrize("scheme", SCHEMES)
def test_dequantize_matches_reference_golden_bitwise(golden, scheme):
    scales = golden[f"{scheme}_scales_f16_bits"].view(np.float16)
    out = convert.dequantize(golden[f"{scheme}_codes"], scales, scheme)
    assert out.tobytes() == golden[f"{scheme}_dequantized"].tobytes()


@pytest.mark.parametrize("threads", [1, 3, 8])
def test_quantize_threads_do_not_change_bits(threads):
    w = convert.normal((64, 512), seed=99, sigma=0.02)
    a = convert.quantize(w, "nf4", threads=1)
    b = convert.quantize(w, "nf4", threads=threads)
    assert a[0].tobytes() == b[0].tobytes() and a[1].tobytes() == b[1].tobytes()


def test_ternary_hand_calculated_bytes_scales_and_half_ties():
    # test_quantization.py:14-23
    weights = np.zeros((2, 128), np.float32)
    weights[0] = np.tile([2, -2, 0, 1], 32)
    codes, scales = convert.quantize(weights, "ternary")
    assert codes.tobytes() == bytes([0x92]) * 32 + bytes([0x55]) * 32
    assert scales.astype("<f2").tobytes() == bytes.fromhex("0040 0000")
    deq = convert.dequantize(codes, scales, "ternary")
    assert deq[0, :4].tolist() == [2, -2, 0, 2]
    assert np.all(deq[1] == 0)


def test_nf4_hand_calculated_nibble_order_and_codebook_roundtrip():
    # test_quantization.py:26-37
    raw = np.tile(np.arange(16, dtype=np.uint8), (2, 8))
    packed = (raw[:, 0::2] | (raw[:, 1::2] << 4)).astype(np.uint8)
    assert packed.tobytes() == bytes.fromhex("10 32 54 76 98 ba dc fe") * 16
    scales = np.array([[1], [2]], np.float16)
    decoded = convert.dequantize(packed, scales, "nf4")
    codes, stored = convert.quantize(decoded[:1], "nf4")
    assert codes.tobytes() == packed[:1].tobytes()
    assert stored.tobytes() == scales[:1].tobytes()


@pytest.mark.parametrize("scheme,zero", [("ternary", 0x55), ("nf4", 0x77)])
def test_zero_and_fp16_underflow_groups(scheme, zero):
    values = np.zeros((2, 128), np.float32)
    values[1] = np.float32(1e-10)
    codes, scales = convert.quantize(values, scheme)
    assert codes.tobytes() == bytes([zero]) * codes.size
    assert np.all(scales == 0)


def test_nf4_ties_choose_lower_index():
    nf4 = np.array([-0.09105003625154495, 0.0, 0.07958029955625534], np.float32)
    values = np.zeros((1, 128), np.float32)
    values[0, 0] = (nf4[1] + nf4[2]) / np.float32(2)
    values[0, 1] = 1
    codes, _ = convert.quantize(values, "nf4")
    assert codes[0, 0] == 0xF7


@pytest.mark.parametrize("scheme", ["ternary", "nf4"])
def test_stored_fp16_scale_is_semantic_value(scheme):
    values = np.zeros((1, 128), np.float32)
    values[0, 0] = 1.0004
    codes, scales = convert.quantize(values, scheme)
    assert scales[0, 0] == np.float16(1)
    assert convert.dequantize(codes, scales, scheme)[0, 0] == np.float32(1)


@pytest.mark.parametrize("values", [
    np.zeros((1, 127)), np.zeros((0, 128)), np.full((1, 128), np.nan),
    np.full((1, 128), 70000.0), np.full((1, 128), np.inf)])
def test_invalid_quantization_inputs(values):
    with pytest.raises(convert.ConversionError):
        convert.quantize(values, "ternary")


def test_f16_conversions_exhaustive_against_numpy():
    from runtime_amd import _ffi

    lib = _ffi.lib()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = convert.f16_to_f32(bits.view(np.float16))
    finite = np.isfinite(want)
    assert got[finite].tobytes() == want[finite].tobytes()
    # f32 -> f16 round-to-nearest-even on a dense sample of f32 bit patterns,
    # including every half-way point between adjacent binary16 values.
    rng = np.random.default_rng(2)
    sample = rng.integers(0, 2**32, size=200000, dtype=np.uint64).astype(np.uint32)
    mids = ((want[finite][:-1].astype(np.float64) + want[finite][1:]) / 2).astype(np.float32)
    f32 = np.concatenate([sample.view(np.float32), mids, np.nextafter(mids, np.float32(np.inf))])
    f32 = f32[np.isfinite(f32)]
    expect = f32.astype(np.float16).view(np.uint16)
    mine = np.array([lib.mfc_f32_to_f16(float(v)) for v in f32[:60000]], np.uint16)
    assert mine.tobytes() == expect[:60000].tobytes()


def test_generator_is_deterministic_and_normal():
    a = convert.normal(100001, seed=0x5EED0001, sigma=0.02, threads=1)
    b = convert.normal(100001, seed=0x5EED0001, sigma=0.02, threads=7)
    assert a.tobytes() == b.tobytes()
    assert abs(float(a.mean())) < 3e-4
    assert abs(float(a.std()) - 0.02) < 3e-4
    c = convert.normal(100001, seed=0x5EED0002, sigma=0.02)
    assert a.tobytes() != c.tobytes()
    ids = convert.token_ids(4096, seed=0x70430001, vocab=65536)
    assert ids.max() < 65536 and len(np.unique(ids)) > 3900
