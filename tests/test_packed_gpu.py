"""GPU parity of the packed-weight operations against the CPU oracle.

Mirrors the reference's hardware-gated suites
(crates/backend-wgpu/tests/parity.rs, int8.rs, packed_pair_validation.rs):
gathers are bitwise, matmuls meet the reference rule
|d| <= 1e-4 + 1e-4*|cpu| (parity.rs:76-87) and max|d|/max|cpu| <= 1e-3,
and every admission reject leaves its outputs untouched.  All calls go
through the C ABI (runtime_amd.backend -> libminifield_hip.so).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle
from runtime_amd import convert
from runtime_amd.backend import WEIGHT, ExecutorError, HipBackend
from tests.conftest import assert_close, max_rel_err

pytestmark = pytest.mark.gpu
SCHEMES = ["ternary", "nf4", "int8"]
# Every product test runs on each kernel path (the `path` fixture): auto
# selects the matrix-core decode GEMV at m <= 8 (activation prologue inside
# the GEMV kernel where it fits); fma forces the FP32-FMA kernels
# everywhere; split runs the matrix-core prologue as a kernel of its own.


def say(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def make_weights(n, k, scheme, seed):
    codes, scales16 = convert.packed_weights(n, k, scheme, seed)
    return codes, convert.f16_to_f32(scales16)


def upload_weights(backend, codes, scales):
    c = backend.upload_u8_classified(codes.shape, codes, WEIGHT)
    s = backend.upload_f32_classified(scales.shape, scales, WEIGHT)
    return c, s


def run_linear(backend, x, codes, scales):
    cb, sb = upload_weights(backend, codes, scales)
    xb = backend.upload_f32(x.shape, x)
    out = backend.allocate_f32((x.shape[0], codes.shape[0]))
    backend.packed_linear(out, xb, cb, sb)
    return backend.read(out)


# --- packed_linear ---------------------------------------------------------------

REFERENCE_SHAPES = [(1, 37, 256), (5, 37, 384), (1, 70000, 128)]  # parity.rs:693-734
NF4_ROWS = [1, 5, 12, 32, 65, 95, 96, 97, 346]                       # parity.rs:1351-1420
INT8_ROWS = [1, 7, 95, 96, 97]                                       # int8.rs:164


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("m,n,k", REFERENCE_SHAPES)
def test_packed_linear_reference_shapes(backend, path, scheme, m, n, k):
    say("packed_linear", scheme, path, m, n, k)
    codes, scales = make_weights(n, k, scheme, 0x5EED0100 + n + k)
    x = convert.normal((m, k), 0xAC70100 + m)
    got = run_linear(backend, x, codes, scales)
    want = oracle.packed_linear(x, codes, scales)
    assert_close(got, want, 1e-4, 1e-4)


@pytest.mark.parametrize("m", NF4_ROWS)
def test_nf4_row_counts(backend, path, m):
    say("nf4 rows", path, m)
    codes, scales = make_weights(96, 1024, "nf4", 0x5EED0200)
    x = convert.normal((m, 1024), 0xAC70200 + m)
    got = run_linear(backend, x, codes, scales)
    assert_close(got, oracle.packed_linear(x, codes, scales), 1e-4, 1e-4)


@pytest.mark.parametrize("m", INT8_ROWS)
def test_int8_rows_match_independent_dense_math(backend, path, m):
    """int8.rs:131-191: signed bytes against dense f64 math, |d| < 0.002."""
    say("int8 rows", path, m)
    rng = np.random.default_rng(m)
    n, k = 64, 384
    codes = rng.integers(-127, 128, size=(n, k), dtype=np.int64).astype(np.int8).view(np.uint8)
    scales = rng.uniform(0.001, 0.01, (n, k // 128)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got = run_linear(backend, x, codes, scales)
    want = oracle.dense_f64(x, oracle.dequantize_f32(codes, scales, "int8"))
    assert np.max(np.abs(got - want)) < 0.002


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("m", [1, 2, 4, 8])
@pytest.mark.parametrize("n,k", [(1024, 1024), (4608, 1024), (2048, 2048), (8192, 2048),
                                 (2048, 8192)])
def test_decode_gemv_sweep_shapes(backend, path, scheme, m, n, k):
    """Decode GEMV over the benchmark sweep shapes (the 65536-row head is
    covered in its own test)."""
    say("gemv sweep", scheme, path, m, n, k)
    codes, scales = make_weights(n, k, scheme, 0x5EED0001 + n + k)
    x = convert.normal((m, k), 0xAC70001 + m)
    got = run_linear(backend, x, codes, scales)
    want = oracle.packed_linear_threaded(x, codes, scales)
    assert max_rel_err(got, want) <= 1e-3
    assert_close(got, want, 1e-4, 1e-4)


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("n,k", [(16384, 2048), (4608, 1024), (1024, 1024), (2048, 8192)])
def test_non_finite_activations_poison_their_rows(backend, path, scheme, n, k):
    """A NaN or infinity in an activation row makes that row's outputs
    non-finite (device backends surface it through argmax rather than a
    per-op check, inference.rs:125-131); the other rows are unaffected."""
    say("non-finite rows", scheme, path, n, k)
    for m in (4, 7):  # one activation fragment, and two (rows 4-7)
        codes, scales = make_weights(n, k, scheme, 0x5EED0300 + n + k)
        x = convert.normal((m, k), 0xAC70300 + k + m)
        x[1, 300] = np.nan
        x[2, 5] = np.inf
        x[3, k - 1] = -np.inf
        bad = [1, 2, 3]
        if m > 4:
            x[5, 77] = np.nan
            x[6, k // 2] = -np.inf
            bad += [5, 6]
        good = [r for r in range(m) if r not in bad]
        got = run_linear(backend, x, codes, scales)
        assert not np.isfinite(got[bad]).any()
        want = oracle.packed_linear_threaded(x[good], codes, scales)
        assert_close(got[good], want, 1e-4, 1e-4)


# Oracle results of the large cases, computed once per (case, inputs) and
# shared by the kernel paths.
_ORACLE_CACHE: dict = {}


def cached_oracle(key, x, codes, scales):
    if key not in _ORACLE_CACHE:
        _ORACLE_CACHE[key] = oracle.packed_linear_threaded(x, codes, scales)
    return _ORACLE_CACHE[key]


_HEAD_WEIGHTS: dict = {}


def head_weights(scheme):
    if scheme not in _HEAD_WEIGHTS:
        _HEAD_WEIGHTS.clear()
        _HEAD_WEIGHTS[scheme] = make_weights(65536, 2048, scheme, 0x5EED0006)
    return _HEAD_WEIGHTS[scheme]


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_lm_head_shape(backend, path, scheme, m):
    """The 65536 x 2048 LM-head shape at every decode batch: the benchmark's
    dominant launch (B = 1), the one- and two-fragment kernels (B <= 4,
    B = 5-8), on every kernel path."""
    say("lm head", scheme, path, m)
    n, k = 65536, 2048
    codes, scales = head_weights(scheme)
    x = convert.normal((m, k), 0xAC70001 + m)
    got = run_linear(backend, x, codes, scales)
    want = cached_oracle(("head", scheme, m), x, codes, scales)
    assert max_rel_err(got, want) <= 1e-3
    assert_close(got, want, 1e-4, 1e-4)


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("m", [1, 2, 3, 8])
@pytest.mark.parametrize("n,k", [(8197, 1024), (12293, 2048), (16384, 1024), (16384, 2048),
                                 (16421, 1024), (16421, 2048), (32773, 1024), (32805, 2048),
                                 (65536, 1024)])
def test_wide_matrix_shapes(backend, path, scheme, m, n, k):
    """At least 513 row tiles at K = 1024 and 2048: the streaming ternary
    kernels (one and two rows, three to eight rows) at 4, 8 and 16 waves per
    block and the streaming NF4 kernel at K = 1024, with row counts that
    leave the last tile partial and the last block short of tiles."""
    say("wide", scheme, path, m, n, k)
    codes, scales = make_weights(n, k, scheme, 0x5EED0007 + n + k)
    x = convert.normal((m, k), 0xAC70011 + m)
    got = run_linear(backend, x, codes, scales)
    want = cached_oracle(("wide", scheme, m, n, k), x, codes, scales)
    assert max_rel_err(got, want) <= 1e-3
    assert_close(got, want, 1e-4, 1e-4)


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("n", [1, 17, 130])
@pytest.mark.parametrize("k", [1024, 2048])
def test_one_row_few_tiles(backend, path, scheme, n, k):
    """One activation row against one, two and nine row tiles (one block of
    K / 256 waves per tile), the last tile partial."""
    say("one row few tiles", scheme, path, n, k)
    codes, scales = make_weights(n, k, scheme, 0x5EED0009 + n + k)
    x = convert.normal((1, k), 0xAC70031 + n + k)
    got = run_linear(backend, x, codes, scales)
    want = oracle.packed_linear(x, codes, scales)
    assert max_rel_err(got, want) <= 1e-3
    assert_close(got, want, 1e-4, 1e-4)


@pytest.mark.parametrize("scheme", ["ternary", "int8"])
@pytest.mark.parametrize("k", [1024, 2048])
@pytest.mark.parametrize("n", [65541, 16421, 2053])
def test_wide_rows_partial_tile_and_row_independence(backend, path, scheme, k, n):
    """Past 4096 row tiles (n = 65541), at 1027 (n = 16421: INT8 on blocks of
    16 waves with several tiles per wave, ternary on the streaming kernels)
    and at 129 row tiles (n = 2053, where each 256-k slice runs as two 128-k
    pieces on two waves), the last tile five rows long: two, five and eight activation rows (dead batch slots in
    the one- and two-fragment layouts) against the oracle, and for INT8
    every row of the batch equal bit for bit to the same row multiplied
    alone (the multi-row wide kernel keeps the one-row kernel's group and
    slice order)."""
    say("wide rows", scheme, path, k, n)
    codes, scales = make_weights(n, k, scheme, 0x5EED0008 + k)
    cb, sb = upload_weights(backend, codes, scales)
    x = convert.normal((8, k), 0xAC70021 + k)
    alone = []
    for b in range(8):
        xb = backend.upload_f32((1, k), x[b:b + 1])
        out = backend.allocate_f32((1, n))
        backend.packed_linear(out, xb, cb, sb)
        alone.append(backend.read(out)[0])
    for m in (2, 5, 8):
        xb = backend.upload_f32((m, k), x[:m])
        out = backend.allocate_f32((m, n))
        backend.packed_linear(out, xb, cb, sb)
        got = backend.read(out)
        want = cached_oracle(("wide rows", scheme, m, n, k), x[:m], codes, scales)
        assert max_rel_err(got, want) <= 1e-3
        assert_close(got, want, 1e-4, 1e-4)
        if path == "auto" and scheme == "int8":
            for b in range(m):
                assert np.array_equal(got[b], alone[b]), (m, b)


def test_int8_k8192_rows_at_a_ragged_width(backend, path):
    """INT8 at K = 8192, two to four rows, 129 row tiles (n = 2053, the last
    tile five rows long; the multi-row wide kernel with sixteen waves of two
    256-k slices each), against the oracle."""
    say("int8 k8192 rows", path)
    n, k = 2053, 8192
    codes, scales = make_weights(n, k, "int8", 0x5EED0031)
    cb, sb = upload_weights(backend, codes, scales)
    x = convert.normal((4, k), 0xAC70031)
    for m in (2, 3, 4):
        xb = backend.upload_f32((m, k), x[:m])
        out = backend.allocate_f32((m, n))
        backend.packed_linear(out, xb, cb, sb)
        got = backend.read(out)
        want = cached_oracle(("int8 k8192", m, n, k), x[:m], codes, scales)
        assert max_rel_err(got, want) <= 1e-3
        assert_close(got, want, 1e-4, 1e-4)


# The prefill GEMM configuration: M in {512, 2048} tokens against 8192 x 2048
# and 2048 x 8192 weights.  M = 512 is checked on every row; M = 2048 on a
# seeded subset of rows (all N columns), the oracle being a scalar CPU path.
_GEMM_WEIGHTS: dict = {}


def gemm_weights(n, k, scheme):
    key = (n, k, scheme)
    if key not in _GEMM_WEIGHTS:
        _GEMM_WEIGHTS.clear()
        _GEMM_WEIGHTS[key] = make_weights(n, k, scheme, 0x5EED0001 + n + k)
    return _GEMM_WEIGHTS[key]


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("n,k", [(8192, 2048), (2048, 8192)])
@pytest.mark.parametrize("m", [512, 2048])
@pytest.mark.parametrize("gemm_path", ["auto", "fma"])
def test_prefill_gemm_config_shapes(backend, gemm_path, scheme, n, k, m):
    say("prefill gemm config", scheme, gemm_path, m, n, k)
    from tests.conftest import PATHS
    codes, scales = gemm_weights(n, k, scheme)
    x = convert.normal((m, k), 0xAC70003 + m)
    previous = backend.set_kernel_path(PATHS[gemm_path])
    try:
        got = run_linear(backend, x, codes, scales)
    finally:
        backend.set_kernel_path(previous)
    if m <= 512:
        rows = np.arange(m)
    else:
        rng = np.random.default_rng(0x6E44 + n + k)
        rows = np.unique(np.concatenate([[0, m - 1], rng.choice(m, 94, replace=False)]))
    want = cached_oracle(("gemm", scheme, n, k, m), x[rows], codes, scales)
    assert np.all(np.isfinite(got))
    assert max_rel_err(got[rows], want) <= 1e-3
    assert_close(got[rows], want, 1e-4, 1e-4)


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("m,n,k", [(512, 8192, 2048), (2048, 8192, 2048), (2048, 4608, 1024)])
@pytest.mark.parametrize("gemm_path", ["auto", "fma"])
def test_prefill_pair_and_swiglu_pair_unsplit(backend, gemm_path, scheme, m, n, k):
    """The two-stream GEMM at the prefill depths where it runs without a
    K split (at least 512 output tiles of 128 x 64 per stream): the FFN
    gate/up pair of both model shapes, in full (all N columns) on a seeded
    subset of rows, against the row-parallel oracle
    (packed_pair_validation.rs:169-208: the pair equals two singles, and
    SwiGLU of the pair equals swiglu_pair, both bitwise in the oracle)."""
    say("prefill pair unsplit", scheme, gemm_path, m, n, k)
    from tests.conftest import PATHS
    ca, sa = make_weights(n, k, scheme, 0x5EED0610 + n + k)
    cb, sb = make_weights(n, k, scheme, 0x5EED0611 + n + k)
    x = convert.normal((m, k), 0xAC70610 + m + k)
    ga, gsa = upload_weights(backend, ca, sa)
    gb, gsb = upload_weights(backend, cb, sb)
    xb = backend.upload_f32(x.shape, x)
    out_a = backend.allocate_f32((m, n))
    out_b = backend.allocate_f32((m, n))
    fused = backend.allocate_f32((m, n))
    previous = backend.set_kernel_path(PATHS[gemm_path])
    try:
        backend.packed_linear_pair(out_a, out_b, xb, ga, gsa, gb, gsb)
        backend.packed_swiglu_pair(fused, xb, ga, gsa, gb, gsb)
        got_a, got_b, got_f = backend.read(out_a), backend.read(out_b), backend.read(fused)
    finally:
        backend.set_kernel_path(previous)
    rng = np.random.default_rng(0x6E46 + m + n + k)
    rows = np.unique(np.concatenate([[0, 127, 128, m - 1], rng.choice(m, 60, replace=False)]))
    want_a = oracle.packed_linear_threaded(x[rows], ca, sa)
    want_b = oracle.packed_linear_threaded(x[rows], cb, sb)
    for got, want in ((got_a, want_a), (got_b, want_b)):
        assert np.all(np.isfinite(got))
        assert max_rel_err(got[rows], want) <= 1e-3
        assert_close(got[rows], want, 1e-4, 1e-4)
    want_f = oracle.swiglu(want_a, want_b)
    assert np.all(np.isfinite(got_f))
    assert max_rel_err(got_f[rows], want_f) <= 1e-3
    assert_close(got_f[rows], want_f, 1e-4, 1e-4)
    for buf in (ga, gsa, gb, gsb, xb, out_a, out_b, fused):
        buf.release()


# --- reserved ternary code 3 ----------------------------------------------------

def test_ternary_reserved_code_decodes_as_plus_two(backend, path):
    """Code 3 is reserved; backend-cpu decodes it as (3 - 1) = +2
    (kernels-simd/src/lib.rs:77-78), and so must every GPU kernel: the
    gather, the decode GEMV (whose tiles store field 3 as (c + 2) mod 4) and
    the prefill GEMM."""
    say("ternary code 3", path)
    rng = np.random.default_rng(0x3333)
    n, k = 320, 1024
    codes = rng.integers(0, 256, size=(n, k // 4), dtype=np.int64).astype(np.uint8)
    codes[:, :8] = 0xFF  # every field 3
    codes[:, 8:16] = 0xC0  # field 3 of the top pair only
    scales = convert.f16_to_f32(rng.uniform(0.001, 0.05, (n, k // 128)).astype(np.float16))
    cb, sb = upload_weights(backend, codes, scales)
    ids = [0, 5, 319, 77]
    out = backend.allocate_f32((len(ids), k))
    backend.packed_gather_rows(out, cb, sb, ids)
    want_rows = oracle.packed_gather_rows(codes, scales, np.array(ids))
    assert backend.read(out).tobytes() == want_rows.tobytes()
    assert np.all(want_rows[:, :32] == 2 * np.repeat(scales[ids, :1], 32, axis=1))
    for m in (1, 5, 100):
        x = convert.normal((m, k), 0xAC70333 + m)
        got = run_linear(backend, x, codes, scales)
        assert_close(got, oracle.packed_linear(x, codes, scales), 1e-4, 1e-4)


# --- wide contractions at one or two rows (f32 vector GEMV) ------------------------
# On the auto path one plain activation row with 4096 <= k <= 8192 (NF4 from
# k = 2048, ternary below 2048 rows from k = 1024) and n <= 8192 runs the f32
# vector GEMV (lanes own 16- or 8-wide k
# slices, waves splitting K); two rows, the other paths and SwiGLU-formed
# activations run the matrix-core or FMA kernels on the same cases.

WIDE_K_SHAPES = [(2048, 8192), (1024, 4608), (1001, 4096), (77, 8192), (8192, 4224), (3, 8192),
                 (1001, 2048), (6144, 3072), (1001, 1024), (2048, 1152)]


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("m", [1, 2])
@pytest.mark.parametrize("n,k", WIDE_K_SHAPES)
def test_wide_k_decode_gemv(backend, path, scheme, m, n, k):
    say("wide k", scheme, path, m, n, k)
    codes, scales = make_weights(n, k, scheme, 0x5EED0500 + n + k)
    x = convert.normal((m, k), 0xAC70500 + m + k)
    got = run_linear(backend, x, codes, scales)
    want = oracle.packed_linear_threaded(x, codes, scales)
    assert_close(got, want, 1e-4, 1e-4)
    assert max_rel_err(got, want) <= 1e-3


@pytest.mark.parametrize("scheme", SCHEMES)
def test_wide_k_f32_scales_and_reserved_codes(backend, path, scheme):
    """Scales that binary16 cannot hold (the kernels then read the f32
    stream), ternary code 3 (+2) and the INT8 extremes +-127, at k = 8192."""
    say("wide k f32 scales", scheme, path)
    rng = np.random.default_rng(0x5151)
    n, k = 640, 8192
    codes, _ = make_weights(n, k, scheme, 0x5EED0510)
    if scheme == "ternary":
        codes[:, :16] = 0xFF
    elif scheme == "int8":
        codes[:, :64] = 0x7F
        codes[:, 64:128] = 0x81
    scales = rng.uniform(0.001, 0.05, (n, k // 128)).astype(np.float32)
    scales[:, 0] = np.float32(0.0123456789)  # not exact in binary16
    for m in (1, 2):
        x = convert.normal((m, k), 0xAC70510 + m)
        got = run_linear(backend, x, codes, scales)
        want = oracle.packed_linear_threaded(x, codes, scales)
        assert_close(got, want, 1e-4, 1e-4)


@pytest.mark.parametrize("scheme", SCHEMES)
def test_wide_k_non_finite_row(backend, path, scheme):
    """A NaN or infinity in one activation row makes all of that row's
    outputs non-finite; the other row matches the oracle."""
    say("wide k non-finite", scheme, path)
    n, k = 512, 8192
    codes, scales = make_weights(n, k, scheme, 0x5EED0520)
    x = convert.normal((2, k), 0xAC70520)
    x[1, 4000] = np.inf
    got = run_linear(backend, x, codes, scales)
    assert not np.isfinite(got[1]).any()
    want = oracle.packed_linear_threaded(x[:1], codes, scales)
    assert_close(got[:1], want, 1e-4, 1e-4)
    x[1, 4000] = np.nan
    got = run_linear(backend, x, codes, scales)
    assert not np.isfinite(got[1]).any()
    # The bad row alone (the one-row kernels).
    assert not np.isfinite(run_linear(backend, x[1:], codes, scales)).any()


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("n,k", [(2048, 8192), (1024, 4608)])
def test_wide_k_swiglu_linear(backend, path, scheme, n, k):
    """packed_swiglu_linear at the FFN down-projection shapes (the
    activations formed by the matrix-core prologue or the staging kernel)."""
    say("wide k swiglu", scheme, path, n, k)
    codes, scales = make_weights(n, k, scheme, 0x5EED0530 + k)
    cb, sb = upload_weights(backend, codes, scales)
    for m in (1, 2):
        gate = convert.normal((m, k), 0xAC70531 + m)
        up = convert.normal((m, k), 0xAC70532 + m)
        gb_ = backend.upload_f32(gate.shape, gate)
        ub_ = backend.upload_f32(up.shape, up)
        out = backend.allocate_f32((m, n))
        backend.packed_swiglu_linear(out, gb_, ub_, cb, sb)
        assert_close(backend.read(out), oracle.packed_swiglu_linear(gate, up, codes, scales))


def test_reference_ternary_fixture_through_the_gpu_gather(backend, golden_dir):
    """crates/executor-core/tests/fixtures/ternary-v1-001: the five rows'
    expected dequantization, bit for bit, from the HIP gather."""
    import json
    doc = json.loads((golden_dir / "ternary-v1-001" / "vectors.json").read_text())
    rows = doc["vectors"]
    codes = np.stack([np.frombuffer(bytes.fromhex(v["expected_codes_hex"]), np.uint8)
                      for v in rows])
    scales16 = np.array([[v["scale_f16"]] for v in rows], dtype=np.float16)
    expected = np.array([v["expected_dequant"] for v in rows], dtype=np.float32)
    cb, sb = upload_weights(backend, codes, convert.f16_to_f32(scales16))
    out = backend.allocate_f32((len(rows), 128))
    backend.packed_gather_rows(out, cb, sb, list(range(len(rows))))
    assert backend.read(out).tobytes() == expected.tobytes()


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("m", [96, 512])
def test_prefill_gemm(backend, path, scheme, m):
    say("prefill gemm", scheme, path, m)
    n, k = 512, 2048
    codes, scales = make_weights(n, k, scheme, 0x5EED0300)
    x = convert.normal((m, k), 0xAC70300 + m)
    got = run_linear(backend, x, codes, scales)
    want = oracle.packed_linear_threaded(x, codes, scales)
    assert max_rel_err(got, want) <= 1e-3
    assert_close(got, want, 1e-4, 1e-4)


# Ragged prefill shapes: partial 128-row and 64-column output tiles, K that
# ends inside a 256-wide ternary chunk, a single group, and shapes where the
# contraction is split across workgroups into 3, 4, 5, 16 and 18 runs of whole
# groups (3 and 5 start runs inside a ternary tile load, which spans two
# groups).
GEMM_EDGE_SHAPES = [(9, 37, 384), (130, 200, 640), (257, 70, 1152), (33, 1000, 128),
                    (129, 4608, 1024), (12, 64, 4096), (100, 1024, 4608), (140, 300, 1920)]


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("m,n,k", GEMM_EDGE_SHAPES)
def test_prefill_gemm_ragged_shapes(backend, path, scheme, m, n, k):
    say("prefill gemm ragged", scheme, path, m, n, k)
    codes, scales = make_weights(n, k, scheme, 0x5EED0310 + n + k)
    x = convert.normal((m, k), 0xAC70310 + m)
    x[m // 2, k // 3] = np.nan
    x[m - 1, 0] = np.inf
    got = run_linear(backend, x, codes, scales)
    want = oracle.packed_linear_threaded(x, codes, scales)
    bad = np.zeros(m, dtype=bool)
    bad[[m // 2, m - 1]] = True
    assert not np.isfinite(got[bad]).any()
    assert max_rel_err(got[~bad], want[~bad]) <= 1e-3
    assert_close(got[~bad], want[~bad], 1e-4, 1e-4)


# --- single-half GEMM activations (opt-in) ----------------------------------------
# mfh_set_gemm_activations(1) keeps one binary16 half of each activation
# (within 2^-12 of itself; absolute 2^-25 of the row's largest below 2^-14 of
# it), so each output is pinned by the a-priori bound
# |d| <= 2^-11 * sum_k |x_k| |w_k| + 1e-6 * max|cpu| (dequantized weights,
# twice the rounding for the sums' own f32 error) and by the normwise rule
# max|d| / max|cpu| <= 1e-3; the per-element 1e-4 rule is the exact default's.

@pytest.fixture
def single_half(backend):
    previous = backend.set_gemm_activations(1)
    yield
    backend.set_gemm_activations(previous)


def _single_half_bound(x, codes, scales, scheme, want):
    w = np.abs(oracle.dequantize_f32(codes, scales, scheme)).astype(np.float64)
    return 2.0 ** -11 * (np.abs(x).astype(np.float64) @ w.T) + 1e-6 * np.max(np.abs(want))


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("m,n,k", [(2048, 8192, 2048), (512, 2048, 8192), (130, 200, 640),
                                   (257, 70, 1152), (33, 1000, 128)])
def test_prefill_gemm_single_half(backend, single_half, scheme, m, n, k):
    say("prefill gemm single half", scheme, m, n, k)
    codes, scales = gemm_weights(n, k, scheme)
    x = convert.normal((m, k), 0xAC70005 + m)
    got = run_linear(backend, x, codes, scales)
    if m <= 512:
        rows = np.arange(m)
    else:
        rng = np.random.default_rng(0x6E45 + n + k)
        rows = np.unique(np.concatenate([[0, m - 1], rng.choice(m, 62, replace=False)]))
    want = oracle.packed_linear_threaded(x[rows], codes, scales)
    assert np.all(np.isfinite(got))
    assert max_rel_err(got[rows], want) <= 1e-3
    diff = np.abs(got[rows].astype(np.float64) - want)
    assert np.all(diff <= _single_half_bound(x[rows], codes, scales, scheme, want))
    # The mode is in effect: the dropped lo halves show at this size.
    assert diff.max() > 1e-6 * np.max(np.abs(want))


@pytest.mark.parametrize("scheme", SCHEMES)
def test_pair_and_swiglu_single_half(backend, single_half, scheme):
    say("pair/swiglu single half", scheme)
    m, n, k = 100, 320, 768
    ca, sa = make_weights(n, k, scheme, 0x5EED0410)
    cb, sb = make_weights(n, k, scheme, 0x5EED0411)
    x = convert.normal((m, k), 0xAC70410)
    ga, gsa = upload_weights(backend, ca, sa)
    gb, gsb = upload_weights(backend, cb, sb)
    xb = backend.upload_f32(x.shape, x)
    out_a = backend.allocate_f32((m, n))
    out_b = backend.allocate_f32((m, n))
    backend.packed_linear_pair(out_a, out_b, xb, ga, gsa, gb, gsb)
    want_a, want_b = oracle.packed_linear_pair(x, ca, sa, cb, sb)
    for got, want, c, s_ in ((backend.read(out_a), want_a, ca, sa),
                             (backend.read(out_b), want_b, cb, sb)):
        assert max_rel_err(got, want) <= 1e-3
        assert np.all(np.abs(got.astype(np.float64) - want) <=
                      _single_half_bound(x, c, s_, scheme, want))
    fused = backend.allocate_f32((m, n))
    backend.packed_swiglu_pair(fused, xb, ga, gsa, gb, gsb)
    assert max_rel_err(backend.read(fused), oracle.packed_swiglu_pair(x, ca, sa, cb, sb)) <= 1e-3


# --- pair / SwiGLU variants -----------------------------------------------------------

@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("m", [1, 3, 8, 100])
def test_pair_and_swiglu_variants(backend, path, scheme, m):
    say("pair/swiglu", scheme, path, m)
    n, k = 320, 768
    ca, sa = make_weights(n, k, scheme, 0x5EED0400)
    cb, sb = make_weights(n, k, scheme, 0x5EED0401)
    x = convert.normal((m, k), 0xAC70400 + m)
    gate = convert.normal((m, k), 0xAC70401 + m)
    up = convert.normal((m, k), 0xAC70402 + m)
    ga, gsa = upload_weights(backend, ca, sa)
    gb, gsb = upload_weights(backend, cb, sb)
    xb = backend.upload_f32(x.shape, x)
    out_a = backend.allocate_f32((m, n))
    out_b = backend.allocate_f32((m, n))
    backend.packed_linear_pair(out_a, out_b, xb, ga, gsa, gb, gsb)
    want_a, want_b = oracle.packed_linear_pair(x, ca, sa, cb, sb)
    assert_close(backend.read(out_a), want_a)
    assert_close(backend.read(out_b), want_b)

    fused = backend.allocate_f32((m, n))
    backend.packed_swiglu_pair(fused, xb, ga, gsa, gb, gsb)
    assert_close(backend.read(fused), oracle.packed_swiglu_pair(x, ca, sa, cb, sb))

    # swiglu_linear contracts over the intermediate width: weights [n2, k].
    n2 = 192
    c2, s2 = make_weights(n2, k, scheme, 0x5EED0402)
    g2, gs2 = upload_weights(backend, c2, s2)
    gb_ = backend.upload_f32(gate.shape, gate)
    ub_ = backend.upload_f32(up.shape, up)
    out = backend.allocate_f32((m, n2))
    backend.packed_swiglu_linear(out, gb_, ub_, g2, gs2)
    assert_close(backend.read(out), oracle.packed_swiglu_linear(gate, up, c2, s2))


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("m", [1, 2, 4])
@pytest.mark.parametrize("n,k", [(8192, 2048), (4608, 1024), (4613, 1024)])
def test_pair_ffn_shape(backend, path, scheme, m, n, k):
    # The LFM2 FFN gate/up shapes (1.2B: 8192 rows per stream at K = 2048;
    # 350M: 4608 at K = 1024; and a partial last tile): one ternary row takes
    # the two-stream wide kernel, more rows the register-prologue plans.
    say("pair ffn shape", scheme, path, m, n, k)
    ca, sa = make_weights(n, k, scheme, 0x5EED0410 + n)
    cb, sb = make_weights(n, k, scheme, 0x5EED0411 + n)
    x = convert.normal((m, k), 0xAC70410 + m)
    ga, gsa = upload_weights(backend, ca, sa)
    gb, gsb = upload_weights(backend, cb, sb)
    xb = backend.upload_f32(x.shape, x)
    out_a = backend.allocate_f32((m, n))
    out_b = backend.allocate_f32((m, n))
    backend.packed_linear_pair(out_a, out_b, xb, ga, gsa, gb, gsb)
    want_a = oracle.packed_linear_threaded(x, ca, sa)
    want_b = oracle.packed_linear_threaded(x, cb, sb)
    assert_close(backend.read(out_a), want_a)
    assert_close(backend.read(out_b), want_b)
    fused = backend.allocate_f32((m, n))
    backend.packed_swiglu_pair(fused, xb, ga, gsa, gb, gsb)
    assert_close(backend.read(fused), oracle.packed_swiglu_pair(x, ca, sa, cb, sb))
    for buf in (ga, gsa, gb, gsb, xb, out_a, out_b, fused):
        buf.release()


# --- gather -----------------------------------------------------------------------

@pytest.mark.parametrize("scheme", SCHEMES)
def test_packed_gather_rows_bitwise(backend, scheme):
    say("gather", scheme)
    rows, k = 64, 384
    codes, scales = make_weights(rows, k, scheme, 0x5EED0500)
    cb, sb = upload_weights(backend, codes, scales)
    ids = [5, 0, 63, 5, 17]
    out = backend.allocate_f32((len(ids), k))
    backend.packed_gather_rows(out, cb, sb, ids)
    want = oracle.packed_gather_rows(codes, scales, np.array(ids))
    assert backend.read(out).tobytes() == want.tobytes()


@pytest.mark.parametrize("scheme", SCHEMES)
def test_device_ids_poison_invalid_rows(backend, scheme):
    say("gather device ids", scheme)
    rows, k = 3, 384
    codes, scales = make_weights(rows, k, scheme, 0x5EED0501)
    cb, sb = upload_weights(backend, codes, scales)
    id_values = np.array([2.0, np.nan, 1.5, -1.0, 3.0, 16777216.0, 0.0], np.float32)
    ids = backend.upload_f32(id_values.shape, id_values)
    out = backend.allocate_f32((id_values.size, k))
    backend.packed_gather_rows(out, cb, sb, ids)
    got = backend.read(out)
    resolved = oracle.resolve_device_ids(id_values)
    resolved[resolved >= rows] = -1  # deferred backends poison out-of-range ids
    want = oracle.packed_gather_rows(codes, scales, resolved)
    for r in range(id_values.size):
        if resolved[r] < 0:
            assert np.all(np.isnan(got[r])), r
        else:
            assert got[r].tobytes() == want[r].tobytes(), r


def test_gather_host_id_out_of_range_and_empty(backend):
    codes, scales = make_weights(4, 128, "ternary", 0x5EED0502)
    cb, sb = upload_weights(backend, codes, scales)
    sentinel = np.full((2, 128), 7.0, np.float32)
    out = backend.upload_f32(sentinel.shape, sentinel)
    with pytest.raises(ExecutorError) as e:
        backend.packed_gather_rows(out, cb, sb, [1, 4])
    assert e.value.variant == "OutOfBounds"
    assert np.array_equal(backend.read(out), sentinel)
    empty = backend.allocate_f32((0, 128))
    backend.packed_gather_rows(empty, cb, sb, [])


# --- admission --------------------------------------------------------------------

def test_rejects_leave_outputs_untouched(backend):
    """packed_pair_validation.rs:57-92: nothing is written on reject."""
    n, k, m = 16, 256, 2
    codes, scales = make_weights(n, k, "ternary", 0x5EED0600)
    cb, sb = upload_weights(backend, codes, scales)
    bad_codes = backend.upload_u8_classified((n, 40), np.zeros((n, 40), np.uint8))
    x = backend.upload_f32((m, k), convert.normal((m, k), 1))
    sentinel = np.full((m, n), -3.0, np.float32)
    out_a = backend.upload_f32(sentinel.shape, sentinel)
    out_b = backend.upload_f32(sentinel.shape, sentinel)
    with pytest.raises(ExecutorError) as e:
        backend.packed_linear_pair(out_a, out_b, x, cb, sb, bad_codes, sb)
    assert e.value.variant == "InvalidShape"
    assert np.array_equal(backend.read(out_a), sentinel)
    assert np.array_equal(backend.read(out_b), sentinel)
    wrong_out = backend.upload_f32((m, n + 1), np.zeros((m, n + 1), np.float32))
    with pytest.raises(ExecutorError) as e:
        backend.packed_linear(wrong_out, x, cb, sb)
    assert e.value.variant == "InvalidShape"
    reserved = np.zeros((n, k), np.uint8)
    reserved[3, 9] = 0x80
    rb = backend.upload_u8_classified(reserved.shape, reserved)
    with pytest.raises(ExecutorError) as e:
        backend.packed_linear(out_a, x, rb, sb)
    assert e.value.variant == "InvalidArgument"
    assert np.array_equal(backend.read(out_a), sentinel)


def test_ownership_and_generation():
    a = HipBackend(0, owner=11)
    b = HipBackend(0, owner=12)
    codes, scales = make_weights(8, 128, "ternary", 0x5EED0700)
    ca, sa = upload_weights(a, codes, scales)
    x = a.upload_f32((1, 128), np.ones((1, 128), np.float32))
    out_b = b.allocate_f32((1, 8))
    with pytest.raises(ExecutorError) as e:
        b.packed_linear(out_b, x, ca, sa)
    assert e.value.variant == "WrongBackend"
    out_a = a.allocate_f32((1, 8))
    a.advance_generation()
    with pytest.raises(ExecutorError) as e:
        a.packed_linear(out_a, x, ca, sa)
    assert e.value.variant == "StaleBuffer"
    a.request_cancel()
    with pytest.raises(ExecutorError) as e:
        a.allocate_f32((4,))
    assert e.value.variant == "Cancelled"
    a.close()
    b.close()


def test_fence_and_readback_completion(backend):
    vals = np.arange(513, dtype=np.float32)
    buf = backend.upload_f32((513,), vals)
    fence = backend.fence()
    while not fence.poll_step():
        pass
    with pytest.raises(ExecutorError) as e:
        fence.poll_step()
    assert e.value.variant == "CompletionConsumed"
    assert np.array_equal(backend.read(buf), vals)
    zeroed = backend.allocate_f32((64,))
    assert np.all(backend.read(zeroed) == 0)
