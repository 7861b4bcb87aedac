"""Pin the CPU oracle before trusting it as the parity reference.

Every oracle function is checked against something independent of its own
loop: the reference's fixture vectors (ternary-v1-001), the kernels-simd and
converter unit-test values, exact closed forms on inputs where every f32
partial sum is exact, exhaustive IEEE binary16 decode against numpy, and f64
brute force.  The `mutant` tests run the same checks against deliberately
broken decoders to show each check catches that class of mistake.
"""
from __future__ import annotations

import json

import numpy as np
import pytest

import oracle
from tests.conftest import max_rel_err

RNG = np.random.default_rng(1234)


def random_codes(n, k, scheme, rng=RNG):
    width = k // oracle.WPB[scheme]
    codes = rng.integers(0, 256, size=(n, width), dtype=np.uint8)
    if scheme == "ternary":
        # keep codes in {0, 1, 2}: clear any 2-bit field equal to 3
        fields = np.stack([(codes >> (2 * j)) & 3 for j in range(4)], -1)
        fields[fields == 3] = 2
        codes = sum((fields[..., j].astype(np.uint8) << (2 * j)) for j in range(4)).astype(np.uint8)
    if scheme == "int8":
        codes[codes == 0x80] = 0x7F
    return codes


# --- fixture: crates/executor-core/tests/fixtures/ternary-v1-001 ----------------

def load_fixture(golden_dir):
    doc = json.loads((golden_dir / "ternary-v1-001" / "vectors.json").read_text())
    rows = doc["vectors"]
    codes = np.stack([np.frombuffer(bytes.fromhex(v["expected_codes_hex"]), np.uint8)
                      for v in rows])
    scales16 = np.array([[v["scale_f16"]] for v in rows], dtype=np.float16)
    expected = np.array([v["expected_dequant"] for v in rows], dtype=np.float32)
    return doc, codes, scales16, expected


def test_fixture_codes_match_expected_code_lists(golden_dir):
    doc, codes, _, _ = load_fixture(golden_dir)
    for row, v in zip(codes, doc["vectors"]):
        unpacked = [(row[j // 4] >> (2 * (j % 4))) & 3 for j in range(128)]
        assert unpacked == v["expected_codes"]


def test_gather_reproduces_fixture_dequant_bitwise(golden_dir):
    _, codes, scales16, expected = load_fixture(golden_dir)
    scales = np.array([[oracle.f16_to_f32(int(b))] for b in scales16.view(np.uint16)[:, 0]],
                      dtype=np.float32)
    out = oracle.packed_gather_rows(codes, scales, np.arange(5))
    assert out.tobytes() == expected.tobytes()


def test_fixture_safetensors_container_matches_vectors(golden_dir):
    from safetensors.numpy import load_file

    tensors = load_file(str(golden_dir / "ternary-v1-001" / "packed.safetensors"))
    _, codes, scales16, expected = load_fixture(golden_dir)
    assert tensors["demo.weight.codes"].tobytes() == codes.tobytes()
    assert tensors["demo.weight.scales"].tobytes() == scales16.tobytes()
    scales = tensors["demo.weight.scales"].astype(np.float32)
    out = oracle.packed_gather_rows(tensors["demo.weight.codes"], scales, np.arange(5))
    assert out.tobytes() == expected.tobytes()


# --- f16 decode: exhaustive against numpy's IEEE conversion -------------------------

def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(want)
    assert got[finite].tobytes() == want[finite].tobytes()
    assert np.all(np.isinf(got[np.isinf(want)]))
    assert np.all(np.isnan(got[np.isnan(want)]))


# --- kernels-simd unit-test invariants (crates/kernels-simd/src/lib.rs:210-268) -----

def test_zero_codes_give_zero_and_minus_one_codes_give_negated_sum():
    x = np.arange(128, dtype=np.float32)
    assert oracle.row_dot("ternary", np.full(32, 0x55, np.uint8), [1.5], x) == 0.0
    got = oracle.row_dot("ternary", np.full(32, 0x00, np.uint8), [2.0], x)
    assert got == np.float32(-2.0 * x.sum())  # integer sums: exact


def test_d2_pattern_group_dot_and_row_accumulation():
    # codes {2,0,1,3} -> weights [1,-1,0,2] repeating (lib.rs:215-228).
    x = ((np.arange(256) - 64.0) * 0.03125).astype(np.float32)  # exact binary fractions
    w = np.tile(np.array([1, -1, 0, 2], np.float64), 64)
    scales = np.array([0.5, 2.0], np.float32)
    want = 0.5 * np.dot(w[:128], x[:128]) + 2.0 * np.dot(w[128:], x[128:])
    got = oracle.row_dot("ternary", np.full(64, 0xD2, np.uint8), scales, x)
    assert got == np.float32(want)  # every partial sum is a multiple of 2^-5: exact


# --- exact closed forms -----------------------------------------------------------

@pytest.mark.parametrize("scheme", ["ternary", "nf4", "int8"])
def test_integer_inputs_match_exact_closed_form(scheme):
    """Small integer activations and power-of-two scales keep every f32 sum
    exact for ternary/int8, so any index, sign or nibble-order mistake
    changes the result."""
    rng = np.random.default_rng(7)
    n, k = 9, 512
    codes = random_codes(n, k, scheme, rng)
    scales = (2.0 ** rng.integers(-2, 3, size=(n, k // 128))).astype(np.float32)
    if scheme == "nf4":
        # one non-zero activation per group: the result is level*x*scale summed
        # over 4 groups of distinct power-of-two magnitude -> still exact when
        # compared in f64 after an f32 rounding of each term.
        x = np.zeros((1, k), np.float32)
        pos = rng.integers(0, 128, size=k // 128) + np.arange(0, k, 128)
        x[0, pos] = 1.0
    else:
        x = rng.integers(-4, 5, size=(3, k)).astype(np.float32)
    dense = oracle.dequantize_f32(codes, scales, scheme).astype(np.float64)
    got = oracle.packed_linear(x, codes, scales)
    want = x.astype(np.float64) @ dense.T
    if scheme == "nf4":
        assert max_rel_err(got, want) < 1e-6
        for r in range(n):
            terms = [np.float32(dense[r, p]) for p in pos]
            acc = np.float32(0)
            for t in terms:
                acc = np.float32(acc + t)
            assert got[0, r] == acc
    else:
        assert np.array_equal(got.astype(np.float64), want)


def test_nf4_even_odd_accumulators_differ_from_sequential_sum():
    """The NF4 group dot keeps separate even/odd accumulators (lib.rs:174-183);
    an input where sequential and split sums round differently tells them
    apart."""
    codes = np.full((1, 64), 0xFF, np.uint8)  # every level = +1.0
    x = np.zeros((1, 128), np.float32)
    x[0, 0] = 1.0
    x[0, 1] = 2.0 ** -24
    x[0, 3] = 2.0 ** -24
    # sequential: ((1 + 2^-24) + 2^-24) = 1 (round to even twice);
    # split: lo = 1, hi = 2^-23 -> 1 + 2^-23 exactly.
    got = oracle.packed_linear(x, codes, np.ones((1, 1), np.float32))
    assert got[0, 0] == np.float32(1.0 + 2.0 ** -23)


# --- brute force on random inputs ----------------------------------------------------

@pytest.mark.parametrize("scheme", ["ternary", "nf4", "int8"])
def test_packed_linear_matches_dense_f64(scheme):
    rng = np.random.default_rng(11)
    n, k, m = 37, 384, 5
    codes = random_codes(n, k, scheme, rng)
    scales = rng.uniform(0.01, 0.1, size=(n, k // 128)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got = oracle.packed_linear(x, codes, scales)
    want = oracle.dense_f64(x, oracle.dequantize_f32(codes, scales, scheme))
    assert max_rel_err(got, want) < 1e-5


@pytest.mark.parametrize("scheme", ["ternary", "nf4", "int8"])
def test_threaded_oracle_is_bitwise_identical(scheme):
    rng = np.random.default_rng(3)
    codes = random_codes(300, 256, scheme, rng)
    scales = rng.uniform(0.01, 0.1, size=(300, 2)).astype(np.float32)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    a = oracle.packed_linear(x, codes, scales)
    b = oracle.packed_linear_threaded(x, codes, scales, threads=7)
    assert a.tobytes() == b.tobytes()


# --- composite ops (backend-cpu/tests/packed_pair_validation.rs:169-208) ---------

@pytest.mark.parametrize("scheme", ["ternary", "nf4", "int8"])
def test_pair_equals_two_singles_and_swiglu_pair_equals_pair_plus_swiglu(scheme):
    rng = np.random.default_rng(5)
    n, k, m = 19, 256, 3
    ca, cb = random_codes(n, k, scheme, rng), random_codes(n, k, scheme, rng)
    sa = rng.uniform(0.01, 0.1, (n, 2)).astype(np.float32)
    sb = rng.uniform(0.01, 0.1, (n, 2)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    a, b = oracle.packed_linear_pair(x, ca, sa, cb, sb)
    assert a.tobytes() == oracle.packed_linear(x, ca, sa).tobytes()
    assert b.tobytes() == oracle.packed_linear(x, cb, sb).tobytes()
    fused = oracle.packed_swiglu_pair(x, ca, sa, cb, sb)
    assert fused.tobytes() == oracle.swiglu(a, b).tobytes()
    gate = rng.standard_normal((m, k)).astype(np.float32)
    up = rng.standard_normal((m, k)).astype(np.float32)
    staged = oracle.packed_swiglu_linear(gate, up, ca, sa)
    assert staged.tobytes() == oracle.packed_linear(oracle.swiglu(gate, up), ca, sa).tobytes()


def test_swiglu_matches_f64_silu():
    g = np.linspace(-20, 20, 1001, dtype=np.float32)
    u = np.linspace(-3, 3, 1001, dtype=np.float32)
    want = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))) * u
    assert max_rel_err(oracle.swiglu(g, u), want) < 1e-6


# --- admission and error behaviour --------------------------------------------------

def test_format_inference_and_rejects():
    s = np.ones((2, 2), np.float32)
    assert oracle.packed_format(np.zeros((2, 64), np.uint8), s) == "ternary"
    assert oracle.packed_format(np.zeros((2, 128), np.uint8), s) == "nf4"
    assert oracle.packed_format(np.zeros((2, 256), np.uint8), s) == "int8"
    with pytest.raises(oracle.OracleError) as e:
        oracle.packed_format(np.zeros((2, 100), np.uint8), s)
    assert e.value.variant == "InvalidShape"
    bad = np.zeros((2, 256), np.uint8)
    bad[1, 7] = 0x80
    with pytest.raises(oracle.OracleError) as e:
        oracle.packed_format(bad, s)
    assert e.value.variant == "InvalidArgument"


def test_non_finite_input_is_backend_failure():
    x = np.zeros((1, 128), np.float32)
    x[0, 3] = np.nan
    with pytest.raises(oracle.OracleError) as e:
        oracle.packed_linear(x, np.zeros((1, 32), np.uint8), np.ones((1, 1), np.float32))
    assert e.value.variant == "BackendFailure"


def test_gather_none_rows_are_nan_and_out_of_range_fails():
    codes = random_codes(4, 256, "ternary")
    scales = np.ones((4, 2), np.float32)
    ids = oracle.resolve_device_ids(np.array([1.0, 2.5, np.inf, -1.0, 3.0, 16777216.0],
                                             np.float32))
    assert ids.tolist() == [1, -1, -1, -1, 3, -1]
    out = oracle.packed_gather_rows(codes, scales, ids)
    assert np.all(np.isnan(out[[1, 2, 3, 5]]))
    assert np.array_equal(out[0], oracle.dequantize_f32(codes, scales, "ternary")[1])
    with pytest.raises(oracle.OracleError) as e:
        oracle.packed_gather_rows(codes, scales, np.array([4]))
    assert e.value.variant == "OutOfBounds"


@pytest.mark.parametrize("scheme", ["ternary", "nf4", "int8"])
def test_gather_equals_level_times_scale(scheme):
    codes = random_codes(6, 384, scheme)
    scales = RNG.uniform(0.01, 2.0, (6, 3)).astype(np.float32)
    out = oracle.packed_gather_rows(codes, scales, np.array([5, 0, 3]))
    want = oracle.dequantize_f32(codes, scales, scheme)[[5, 0, 3]]
    assert out.tobytes() == want.tobytes()


# --- the checks catch plausible mistakes --------------------------------------------

def _nf4_high_nibble_first(codes, scales):
    q = np.stack([codes >> 4, codes & 15], -1).reshape(codes.shape[0], -1)
    return oracle.NF4_LEVELS[q] * np.repeat(scales, 128, axis=1)


def _ternary_msb_first(codes, scales):
    q = np.stack([(codes >> (6 - 2 * j)) & 3 for j in range(4)], -1).reshape(codes.shape[0], -1)
    return (q.astype(np.float32) - 1) * np.repeat(scales, 128, axis=1)


def _ternary_code_minus_two(codes, scales):
    q = np.stack([(codes >> (2 * j)) & 3 for j in range(4)], -1).reshape(codes.shape[0], -1)
    return (q.astype(np.float32) - 2) * np.repeat(scales, 128, axis=1)


def _int8_unsigned(codes, scales):
    return codes.astype(np.float32) * np.repeat(scales, 128, axis=1)


@pytest.mark.parametrize("mutant", [_nf4_high_nibble_first, _ternary_msb_first,
                                    _ternary_code_minus_two, _int8_unsigned])
def test_fixture_check_rejects_mutant_decoders(golden_dir, mutant):
    """The fixture and closed-form checks above fail for decoders with a
    swapped nibble/bit order, a wrong offset or a lost sign."""
    _, codes, scales16, expected = load_fixture(golden_dir)
    scales = scales16.astype(np.float32)
    if mutant is _nf4_high_nibble_first:
        raw = np.tile(np.arange(16, dtype=np.uint8), (1, 8))
        packed = (raw[:, 0::2] | (raw[:, 1::2] << 4)).astype(np.uint8)
        want = np.tile(oracle.NF4_LEVELS, 8)[None]
        assert not np.array_equal(mutant(packed, np.ones((1, 1), np.float32)), want)
        assert np.array_equal(oracle.packed_gather_rows(packed, np.ones((1, 1), np.float32),
                                                        [0]), want)
    elif mutant is _int8_unsigned:
        codes8 = np.array([[0xFF] * 128], np.uint8)
        assert not np.array_equal(mutant(codes8, np.ones((1, 1), np.float32)),
                                  oracle.packed_gather_rows(codes8, np.ones((1, 1), np.float32),
                                                            [0]))
    else:
        assert not np.array_equal(mutant(codes, scales), expected)
