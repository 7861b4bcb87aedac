"""GPU parity of the dense LFM2 operations (runtime_amd/csrc/dense.hip).

Every call goes through the C ABI.  Three kinds of check, as the
reference's own suites do (crates/backend-cpu/tests/model_ops_fixture.rs,
inference_ops_fixture.rs, crates/backend-wgpu/tests/parity.rs):
  * the reference's fixture cases within their stated tolerance;
  * the oracle on seeded inputs at LFM2 shapes: bitwise where the kernel
    keeps the reference's exact arithmetic (copies, gathers, selectors,
    element-wise, rotary, the convolution, cache appends), otherwise the
    reference's device rule |d| <= 1e-4 + 1e-4 * |cpu|;
  * admission: the reference's status and message, outputs untouched.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle
from dense_fixtures import (close, conv_operands, f32, gqa_operands, head_rms_operands,
                            inference_operands, inference_ops_cases, model_ops_cases,
                            rotary_operands, sentinels)
from runtime_amd.backend import (CacheLength, ExecutorError, GatedShortConvSpec, GqaSpec,
                                 PackedHeadSpec, RectCopy2d, RotarySpec)
from tests.conftest import assert_close, max_rel_err

pytestmark = pytest.mark.gpu


def say(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def rng_f32(seed, shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def up(backend, a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return backend.upload_f32(a.shape, a)


def bits_equal(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---- the reference's fixtures ------------------------------------------------

def run_conv(backend, projection, kernel, history, hidden, width):
    hb = up(backend, history)
    out = backend.allocate_f32((projection.shape[0], hidden))
    backend.gated_short_convolution(out, up(backend, projection), up(backend, kernel), hb,
                                    GatedShortConvSpec(hidden, width))
    return backend.read(out), backend.read(hb)


def run_gqa(backend, q, k, v, kc, vc, start, qh, kvh, d):
    kcb, vcb = up(backend, kc), up(backend, vc)
    out = backend.allocate_f32(q.shape)
    length = CacheLength(start)
    backend.causal_gqa(out, up(backend, q), up(backend, k), up(backend, v), kcb, vcb, length,
                       GqaSpec(qh, kvh, d))
    return backend.read(out), backend.read(kcb), backend.read(vcb), length.value


@pytest.mark.parametrize("case", model_ops_cases(), ids=lambda c: c["id"])
def test_model_ops_fixture(backend, case):
    say("model-ops", case["id"])
    op = case["operation"]
    if op == "gated_short_convolution":
        projection, kernel, history, hidden, width, expected, tail = conv_operands(case)
        out, hist = run_conv(backend, projection, kernel, history, hidden, width)
        assert close(out, expected)
        flat = hist.reshape(-1)
        assert close(flat[flat.size - tail.size:], tail)
    elif op == "split_half_rotary":
        x, positions, heads, dim, theta, expected = rotary_operands(case)
        out = backend.allocate_f32(x.shape)
        backend.split_half_rotary(out, up(backend, x), positions,
                                  RotarySpec(PackedHeadSpec(heads, dim), theta))
        assert close(backend.read(out), expected)
    elif op == "head_local_rms":
        x, weight, heads, dim, eps, expected = head_rms_operands(case)
        out = backend.allocate_f32(x.shape)
        backend.head_rms_norm(out, up(backend, x), up(backend, weight), PackedHeadSpec(heads, dim),
                              eps)
        assert close(backend.read(out), expected)
    else:
        o = gqa_operands(case)
        out, kc, vc, length = run_gqa(backend, o["query"], o["key"], o["value"], o["key_cache"],
                                      o["value_cache"], o["cache_len"], o["query_heads"],
                                      o["kv_heads"], o["head_dim"])
        assert length == o["all_keys"].shape[0]
        assert close(out, o["expected"])
        assert np.array_equal(kc, o["all_keys"]) and np.array_equal(vc, o["all_values"])


@pytest.mark.parametrize("case", inference_ops_cases(), ids=lambda c: c["id"])
def test_inference_ops_fixture(backend, case):
    say("inference-ops", case["id"])
    o = inference_operands(case)
    op = case["operation"]
    exp = o["expected"]
    out = backend.allocate_f32(exp.shape)
    if op == "linear":
        backend.linear(out, up(backend, o["x"]), up(backend, o["weight"]))
    elif op == "rms_norm":
        backend.row_rms_norm(out, up(backend, o["x"]), up(backend, o["weight"]),
                             np.float32(o["epsilon_f32"]))
    elif op == "embedding":
        backend.gather_rows(out, up(backend, o["weight"]), o["token_ids"])
    elif op == "swiglu":
        backend.swiglu(out, up(backend, o["gate"]), up(backend, o["up"]))
    elif op == "add":
        backend.add(out, up(backend, o["left"]), up(backend, o["right"]))
    else:
        backend.multiply(out, up(backend, o["left"]), up(backend, o["right"]))
    assert close(backend.read(out), exp)


def test_rotary_sentinel_bits(backend):
    s = sentinels()["rotary"]
    x = f32(s["input"]).reshape(1, 2)
    out = backend.allocate_f32((1, 2))
    backend.split_half_rotary(out, up(backend, x), [s["position"]],
                              RotarySpec(PackedHeadSpec(1, s["head_dim"]), np.float32(s["theta"])))
    assert backend.read(out).view(np.uint32).reshape(-1).tolist() == s["expected_u32"]


def test_conv_sentinel_bits(backend):
    s = sentinels()["convolution"]
    projection = np.concatenate([f32(s["B"]), f32(s["C"]), f32(s["V"])], axis=1)
    kernel = f32(s["kernel"])
    out, _ = run_conv(backend, projection, kernel, f32(s["prefix_U"]), 1, kernel.shape[1])
    assert out.view(np.uint32).reshape(-1).tolist() == np.asarray(
        s["expected_u32"]).reshape(-1).tolist()


# ---- oracle parity at LFM2 shapes ----------------------------------------------

@pytest.mark.parametrize("rows,width", [(1, 1), (1, 1024), (7, 2048), (3, 65), (130, 512),
                                        (2, 5000)])
def test_row_rms_norm(backend, rows, width):
    say("row_rms_norm", rows, width)
    x = rng_f32(10 + width, (rows, width))
    w = rng_f32(11 + width, (width,))
    out = backend.allocate_f32(x.shape)
    backend.row_rms_norm(out, up(backend, x), up(backend, w), np.float32(1e-5))
    assert_close(backend.read(out), oracle.row_rms_norm(x, w, np.float32(1e-5)))


@pytest.mark.parametrize("rows,width", [(1, 1024), (4, 2048), (9, 333)])
def test_add_row_rms_norm(backend, rows, width):
    say("add_row_rms_norm", rows, width)
    left, right = rng_f32(20, (rows, width)), rng_f32(21, (rows, width))
    w = rng_f32(22, (width,))
    total, normed = backend.allocate_f32(left.shape), backend.allocate_f32(left.shape)
    backend.add_row_rms_norm(total, normed, up(backend, left), up(backend, right), up(backend, w),
                             np.float32(1e-5))
    want_sum, want_norm = oracle.add_row_rms_norm(left, right, w, np.float32(1e-5))
    assert bits_equal(backend.read(total), want_sum)
    assert_close(backend.read(normed), want_norm)


@pytest.mark.parametrize("tokens,heads,dim", [(1, 16, 64), (9, 8, 64), (3, 2, 200), (2, 3, 6)])
def test_head_rms_norm(backend, tokens, heads, dim):
    say("head_rms_norm", tokens, heads, dim)
    x = rng_f32(30, (tokens, heads * dim))
    w = rng_f32(31, (dim,))
    out = backend.allocate_f32(x.shape)
    backend.head_rms_norm(out, up(backend, x), up(backend, w), PackedHeadSpec(heads, dim),
                          np.float32(1e-5))
    assert_close(backend.read(out), oracle.head_rms_norm(x, w, heads, dim, np.float32(1e-5)))


@pytest.mark.parametrize("tokens,heads,dim,theta", [(1, 32, 64, 1e6), (5, 8, 64, 1e6),
                                                    (3, 2, 6, 1e4), (4, 1, 130, 5e5)])
def test_split_half_rotary_bitwise(backend, tokens, heads, dim, theta):
    say("split_half_rotary", tokens, heads, dim)
    x = rng_f32(40, (tokens, heads * dim))
    positions = np.array([0, 1, 31, 4095, 127999][:tokens] + [7] * max(0, tokens - 5),
                         dtype=np.uint64)
    out = backend.allocate_f32(x.shape)
    backend.split_half_rotary(out, up(backend, x), positions,
                              RotarySpec(PackedHeadSpec(heads, dim), np.float32(theta)))
    want = oracle.split_half_rotary(x, positions, heads, dim, np.float32(theta))
    assert bits_equal(backend.read(out), want)


@pytest.mark.parametrize("base", [0, 2047, (1 << 24) - 2, (1 << 40) + 3])
def test_rotary_consecutive_positions_bitwise(backend, base):
    # Consecutive positions travel as a base in the kernel arguments; the
    # device's u64 -> f32 conversion must round as the host's does (2^24 + 1
    # rounds to 2^24 here).
    say("rotary consecutive", base)
    tokens, heads, dim = 4, 3, 64
    x = rng_f32(45, (tokens, heads * dim))
    positions = np.arange(base, base + tokens, dtype=np.uint64)
    out = backend.allocate_f32(x.shape)
    backend.split_half_rotary(out, up(backend, x), positions,
                              RotarySpec(PackedHeadSpec(heads, dim), np.float32(1e6)))
    want = oracle.split_half_rotary(x, positions, heads, dim, np.float32(1e6))
    assert bits_equal(backend.read(out), want)


@pytest.mark.parametrize("consecutive", [True, False])
@pytest.mark.parametrize("tokens,qh,kvh,dim", [(1, 32, 8, 64), (1, 16, 8, 64), (6, 4, 2, 8)])
def test_qk_norm_rope(backend, tokens, qh, kvh, dim, consecutive):
    say("qk_norm_rope", tokens, qh, kvh, dim, consecutive)
    q, k = rng_f32(50, (tokens, qh * dim)), rng_f32(51, (tokens, kvh * dim))
    qw, kw = rng_f32(52, (dim,)), rng_f32(53, (dim,))
    positions = np.arange(100, 100 + tokens, dtype=np.uint64)
    if not consecutive:
        positions = (positions * 7 + 3)[::-1].copy()
    q_out, k_out = backend.allocate_f32(q.shape), backend.allocate_f32(k.shape)
    backend.qk_norm_rope(q_out, k_out, up(backend, q), up(backend, k), up(backend, qw),
                         up(backend, kw), positions,
                         RotarySpec(PackedHeadSpec(qh, dim), np.float32(1e6)),
                         PackedHeadSpec(kvh, dim), np.float32(1e-5))
    want_q, want_k = oracle.qk_norm_rope(q, k, qw, kw, positions, qh, kvh, dim,
                                         np.float32(1e6), np.float32(1e-5))
    assert_close(backend.read(q_out), want_q)
    assert_close(backend.read(k_out), want_k)


GQA_CASES = [
    # tokens, start, capacity, query heads, kv heads, head_dim
    (1, 0, 8, 32, 8, 64),
    (1, 5, 8, 32, 8, 64),
    (1, 300, 512, 16, 8, 64),
    (1, 1500, 2048, 32, 8, 64),     # crosses the 1024-key chunk
    (17, 0, 32, 32, 8, 64),
    (17, 40, 64, 16, 8, 64),
    (3, 2, 8, 6, 2, 2),
    (2, 3, 8, 4, 2, 96),             # head wider than a wave, two key groups
    (2, 3, 8, 2, 1, 256),
    (2, 3, 8, 2, 2, 320),            # two dimensions per thread
    # split-key path (few (token, head) pairs over more than 64 keys)
    (4, 700, 1024, 32, 8, 64),
    (1, 3000, 4096, 6, 2, 128),      # LDS too large for the split path
    (1, 600, 1024, 8, 1, 64),
    (2, 513, 1024, 16, 2, 256),      # LDS too large for the split path
    (1, 64, 128, 4, 4, 32),          # two ranges, the last holding one key
    (1, 200, 256, 16, 8, 64),        # ragged last range
    (3, 130, 256, 8, 2, 96),         # group of four, 96-wide heads
    (1, 2500, 2561, 32, 8, 64),      # decode at the end of a 2048-token prefill
    # prefill on the fp32 matrix-core kernel (64-row tiles, 64-key tiles)
    (130, 0, 256, 32, 8, 64),        # ragged last token tile and key tile
    (300, 50, 512, 16, 8, 64),       # cached prefix, tiles straddling it
    (64, 0, 64, 2, 1, 112),          # widest head of the path, one key tile
    (200, 7, 256, 6, 2, 16),         # group of three: 64-row tiles hold 21 tokens
    (130, 1000, 1200, 8, 8, 32),     # group of one over a long cached prefix
    (40, 3, 64, 20, 4, 48),          # group of five
    (33, 0, 40, 64, 1, 80),          # group of 64: one token per block
    (512, 0, 512, 32, 8, 64),        # the LFM2-1.2B head layout
]


@pytest.mark.parametrize("tokens,start,cap,qh,kvh,d", GQA_CASES)
def test_causal_gqa(backend, tokens, start, cap, qh, kvh, d):
    say("causal_gqa", tokens, start, cap, qh, kvh, d)
    seed = tokens * 1000 + start + d
    q = rng_f32(seed, (tokens, qh * d))
    k, v = rng_f32(seed + 1, (tokens, kvh * d)), rng_f32(seed + 2, (tokens, kvh * d))
    kc, vc = rng_f32(seed + 3, (cap, kvh * d)), rng_f32(seed + 4, (cap, kvh * d))
    out, kc2, vc2, length = run_gqa(backend, q, k, v, kc, vc, start, qh, kvh, d)
    want, want_kc, want_vc, want_len = oracle.causal_gqa(q, k, v, kc, vc, start, qh, kvh, d)
    assert length == want_len == start + tokens
    assert_close(out, want)
    assert bits_equal(kc2, want_kc) and bits_equal(vc2, want_vc)


def test_causal_gqa_prefill_at_2048_tokens(backend):
    """The 1.2B-shape prefill attention at its full depth: 2048 tokens of
    32 query / 8 key-value heads of width 64 on an empty cache, against the
    score-cached oracle (bitwise equal to the literal restatement, since
    gqa_score is pure: attention_convolution.rs:190-216)."""
    tokens, qh, kvh, d = 2048, 32, 8, 64
    say("causal_gqa prefill", tokens, qh, kvh, d)
    seed = 0x6A2048
    q = rng_f32(seed, (tokens, qh * d))
    k, v = rng_f32(seed + 1, (tokens, kvh * d)), rng_f32(seed + 2, (tokens, kvh * d))
    kc = np.zeros((tokens, kvh * d), dtype=np.float32)
    vc = np.zeros((tokens, kvh * d), dtype=np.float32)
    out, kc2, vc2, length = run_gqa(backend, q, k, v, kc, vc, 0, qh, kvh, d)
    want, want_kc, want_vc, want_len = oracle.causal_gqa(q, k, v, kc, vc, 0, qh, kvh, d,
                                                         threads=16)
    assert length == want_len == tokens
    assert max_rel_err(out, want) <= 1e-3
    assert_close(out, want)
    assert bits_equal(kc2, want_kc) and bits_equal(vc2, want_vc)


@pytest.mark.parametrize("tokens,hidden,width", [(1, 1024, 3), (1, 2048, 3), (7, 2053, 3),
                                                 (1, 64, 1), (2, 100, 4), (5, 16, 2), (1, 1, 3),
                                                 # (token, channel) threads + separate roll
                                                 (17, 2048, 3), (300, 1000, 3), (2048, 2048, 3),
                                                 (20, 33, 25), (40, 7, 1)])
def test_gated_short_convolution_bitwise(backend, tokens, hidden, width):
    say("gated_short_convolution", tokens, hidden, width)
    projection = rng_f32(60 + tokens, (tokens, 3 * hidden))
    kernel = rng_f32(61, (hidden, width))
    history = rng_f32(62, (width - 1, hidden))
    out, hist = run_conv(backend, projection, kernel, history, hidden, width)
    want, want_hist = oracle.gated_short_convolution(projection, kernel, history, hidden, width)
    assert bits_equal(out, want)
    assert bits_equal(hist, want_hist)


def test_conv_decode_steps_roll_history(backend):
    # Token-by-token decoding equals one prefill over the same tokens.
    hidden, width, tokens = 48, 3, 6
    projection = rng_f32(70, (tokens, 3 * hidden))
    kernel = rng_f32(71, (hidden, width))
    history0 = np.zeros((width - 1, hidden), dtype=np.float32)
    full, full_hist = oracle.gated_short_convolution(projection, kernel, history0, hidden, width)
    hb = up(backend, history0)
    kb = up(backend, kernel)
    rows = []
    for t in range(tokens):
        out = backend.allocate_f32((1, hidden))
        backend.gated_short_convolution(out, up(backend, projection[t:t + 1]), kb, hb,
                                        GatedShortConvSpec(hidden, width))
        rows.append(backend.read(out))
    assert bits_equal(np.concatenate(rows), full)
    assert bits_equal(backend.read(hb), full_hist)


@pytest.mark.parametrize("rows,width", [(1, 1), (1, 1000), (1, 65536), (3, 65537), (64, 300)])
def test_argmax(backend, rows, width):
    say("argmax", rows, width)
    x = np.random.default_rng(80 + width).integers(-50, 50, size=(rows, width)).astype(np.float32)
    out = backend.allocate_f32((rows,))
    backend.argmax(out, up(backend, x))
    assert bits_equal(backend.read(out), oracle.argmax(x))


def test_argmax_poison_and_ties(backend):
    x = np.zeros((4, 2000), dtype=np.float32)
    x[0, 1500] = 3.0
    x[0, 1999] = 3.0                   # tie: first index wins
    x[1, 7] = np.nan
    x[2, 1999] = -np.inf
    x[3, :] = -1.0                     # all equal: index 0
    out = backend.allocate_f32((4,))
    backend.argmax(out, up(backend, x))
    got = backend.read(out)
    assert got[0] == 1500 and np.isnan(got[1]) and np.isnan(got[2]) and got[3] == 0
    assert bits_equal(got, oracle.argmax(x))


def test_argmax_wide_rows_ties_and_poison(backend):
    # Wide rows are scanned in ranges by separate blocks: ties across ranges
    # keep the lower index and a NaN in any range poisons the row.
    x = np.zeros((3, 40000), dtype=np.float32)
    x[0, 9000] = x[0, 30000] = 5.0
    x[1, 39999] = np.nan
    x[2, 12345] = -np.inf
    x[2, 20000] = 1.0
    out = backend.allocate_f32((3,))
    backend.argmax(out, up(backend, x))
    got = backend.read(out)
    assert got[0] == 9000 and np.isnan(got[1]) and np.isnan(got[2])
    assert bits_equal(got, oracle.argmax(x))


def test_argmax_wider_than_64_ranges(backend):
    # Past 64 ranges of 2048 (131072 entries) the range winners no longer fit
    # one lane each of the final wave.
    width = 140000
    x = np.random.default_rng(0xA86).integers(-50, 50, size=(4, width)).astype(np.float32)
    x[0, 1000] = x[0, 139000] = 99.0   # tie across the first and the last range
    x[1, 135000] = np.nan              # poison past 131072
    x[2, 131072] = 100.0               # the unique maximum, first entry past 64 ranges
    x[3, :] = 7.0                      # all equal: index 0
    out = backend.allocate_f32((4,))
    backend.argmax(out, up(backend, x))
    got = backend.read(out)
    assert got[0] == 1000 and np.isnan(got[1]) and got[2] == 131072 and got[3] == 0
    assert bits_equal(got, oracle.argmax(x))


@pytest.mark.parametrize("width", [1, 64, 130, 65536])
def test_argmax_masked(backend, width):
    say("argmax_masked", width)
    rng = np.random.default_rng(90 + width)
    x = rng.integers(-20, 20, size=(3, width)).astype(np.float32)
    allowed = rng.random(width) < 0.25
    allowed[0] = True
    words = np.zeros((width + 63) // 64, dtype=np.uint64)
    for i in np.nonzero(allowed)[0]:
        words[i // 64] |= np.uint64(1) << np.uint64(i % 64)
    x[1, ~allowed] = np.nan          # masked-out NaN does not poison
    out = backend.allocate_f32((3,))
    backend.argmax_masked(out, up(backend, x), words)
    assert bits_equal(backend.read(out), oracle.argmax(x, words))
    backend.argmax_masked(out, up(backend, x), np.zeros_like(words))
    assert np.all(np.isnan(backend.read(out)))


def test_gather_rows_host_and_device_ids(backend):
    table = rng_f32(100, (50, 1024))
    tb = up(backend, table)
    ids = [49, 0, 7, 7, 13]
    out = backend.allocate_f32((len(ids), 1024))
    backend.gather_rows(out, tb, ids)
    assert bits_equal(backend.read(out), table[ids])
    # Device ids: invalid selectors give NaN rows (as the oracle's None), and
    # an in-range id past the table also gives a NaN row on the device.
    dev = np.array([3.0, -1.0, 2.5, np.nan, 16777216.0, 49.0, 50.0], dtype=np.float32)
    out = backend.allocate_f32((dev.size, 1024))
    backend.gather_rows(out, tb, up(backend, dev))
    got = backend.read(out)
    resolved = oracle.resolve_device_ids(dev)
    resolved[resolved >= 50] = -1
    assert bits_equal(got, oracle.gather_rows(table, resolved))


def test_gather_columns(backend):
    x = rng_f32(110, (6, 300))
    cols = [299, 0, 5, 5, 120]
    out = backend.allocate_f32((6, len(cols)))
    backend.gather_columns(out, up(backend, x), cols)
    assert bits_equal(backend.read(out), oracle.gather_columns(x, cols))


@pytest.mark.parametrize("count", [1, 3, 4, 4099, 1 << 20])
def test_copy_add_multiply_bitwise(backend, count):
    left, right = rng_f32(120, (count,)), rng_f32(121, (count,))
    lb, rb = up(backend, left), up(backend, right)
    out = backend.allocate_f32((count,))
    backend.copy(out, lb)
    assert bits_equal(backend.read(out), left)
    backend.add(out, lb, rb)
    assert bits_equal(backend.read(out), oracle.add(left, right))
    backend.multiply(out, lb, rb)
    assert bits_equal(backend.read(out), oracle.multiply(left, right))


def test_copy_rect_2d(backend):
    # model_ops_fixture.rs:355-381.
    src = np.arange(12, dtype=np.float32).reshape(3, 4)
    dst = np.full((4, 5), -1.0, dtype=np.float32)
    db = up(backend, dst)
    backend.copy_rect_2d(db, up(backend, src), RectCopy2d(1, 1, 2, 2, 2, 3))
    assert bits_equal(backend.read(db), oracle.copy_rect_2d(dst, src, (1, 1, 2, 2, 2, 3)))
    assert backend.read(db).reshape(-1).tolist() == [
        -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, 5, 6, 7, -1, -1, 9, 10, 11]
    with pytest.raises(ExecutorError) as info:
        backend.copy_rect_2d(db, up(backend, src), RectCopy2d(2, 3, 0, 0, 2, 1))
    assert info.value.variant == "OutOfBounds"


@pytest.mark.parametrize("count", [10, 1 << 16])
def test_swiglu(backend, count):
    gate, upv = rng_f32(130, (1, count), 4.0), rng_f32(131, (1, count))
    out = backend.allocate_f32((1, count))
    backend.swiglu(out, up(backend, gate), up(backend, upv))
    assert_close(backend.read(out), oracle.swiglu(gate, upv))


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (3, 17, 300), (8, 64, 2048)])
def test_linear(backend, m, n, k):
    x, w = rng_f32(140, (m, k)), rng_f32(141, (n, k), 0.05)
    out = backend.allocate_f32((m, n))
    backend.linear(out, up(backend, x), up(backend, w))
    assert_close(backend.read(out), oracle.linear(x, w))


# ---- admission ------------------------------------------------------------------

def expect_error(variant, message, fn, *args):
    with pytest.raises(ExecutorError) as info:
        fn(*args)
    assert info.value.variant == variant, info.value
    assert info.value.message == message, info.value


def test_dense_admission_matches_reference(backend):
    b = backend
    x = up(b, np.ones((2, 8), dtype=np.float32))
    w8 = up(b, np.ones(8, dtype=np.float32))
    sentinel = np.full((2, 8), 7.0, dtype=np.float32)
    out = up(b, sentinel)
    expect_error("InvalidArgument", "RMS epsilon must be finite and positive",
                 b.row_rms_norm, out, x, w8, np.float32(0.0))
    expect_error("InvalidShape", "RMS input width differs from weight width",
                 b.row_rms_norm, out, x, up(b, np.ones(4, dtype=np.float32)), np.float32(1e-5))
    expect_error("InvalidArgument", "head count and head dimension must be nonzero",
                 b.head_rms_norm, out, x, w8, PackedHeadSpec(0, 8), np.float32(1e-5))
    expect_error("InvalidShape", "packed head tensor width differs from descriptor",
                 b.head_rms_norm, out, x, w8, PackedHeadSpec(3, 8), np.float32(1e-5))
    expect_error("InvalidShape", "split-half RoPE requires an even head dimension",
                 b.split_half_rotary, out, x, [0, 1], RotarySpec(PackedHeadSpec(8, 1), 1e4))
    expect_error("InvalidArgument", "RoPE theta must be finite and positive",
                 b.split_half_rotary, out, x, [0, 1], RotarySpec(PackedHeadSpec(2, 4), -1.0))
    expect_error("InvalidShape", "RoPE position count differs from token count",
                 b.split_half_rotary, out, x, [0], RotarySpec(PackedHeadSpec(2, 4), 1e4))
    expect_error("InvalidShape", "elementwise operands have different layouts",
                 b.add, out, x, up(b, np.ones((8, 2), dtype=np.float32)))
    expect_error("InvalidShape", "output layout differs from required contiguous shape",
                 b.add, up(b, np.ones((2, 9), dtype=np.float32)), x, x)
    expect_error("InvalidArgument", "output aliases an input", b.add, x, x, x)
    expect_error("Unsupported",
                 "rectangular copy does not permit overlapping source and destination allocation",
                 b.copy_rect_2d, x, x, RectCopy2d(0, 0, 0, 0, 1, 1))
    expect_error("InvalidShape", "linear input width differs from weight width",
                 b.linear, out, x, up(b, np.ones((8, 4), dtype=np.float32)))
    expect_error("OutOfBounds", "gather identifier exceeds row count",
                 b.gather_rows, up(b, np.zeros((1, 8), dtype=np.float32)), x, [2])
    expect_error("OutOfBounds", "column gather identifier exceeds input width",
                 b.gather_columns, up(b, np.zeros((2, 1), dtype=np.float32)), x, [8])
    expect_error("InvalidArgument", "masked argmax mask length must be ceil(width / 64)",
                 b.argmax_masked, up(b, np.zeros(2, dtype=np.float32)), x, [1, 1])
    expect_error("InvalidShape", "SwiGLU gate and up layouts differ",
                 b.swiglu, out, x, up(b, np.ones((1, 16), dtype=np.float32)))
    assert bits_equal(b.read(out), sentinel)


def test_gqa_rejects_over_capacity_before_mutating(backend):
    # model_ops_fixture.rs:383-430.
    b = backend
    q = up(b, np.array([[0.1, 0.2, 0.3, 0.4]], dtype=np.float32))
    k = up(b, np.array([[0.5, 0.6]], dtype=np.float32))
    v = up(b, np.array([[0.7, 0.8]], dtype=np.float32))
    kc = up(b, np.array([[1, 2], [3, 4]], dtype=np.float32))
    vc = up(b, np.array([[5, 6], [7, 8]], dtype=np.float32))
    out = up(b, np.full((1, 4), 9.0, dtype=np.float32))
    length = CacheLength(2)
    expect_error("OutOfBounds", "GQA append exceeds cache capacity",
                 b.causal_gqa, out, q, k, v, kc, vc, length, GqaSpec(2, 1, 2))
    assert length.value == 2
    assert b.read(kc).tolist() == [[1, 2], [3, 4]] and b.read(vc).tolist() == [[5, 6], [7, 8]]
    assert b.read(out).tolist() == [[9, 9, 9, 9]]
    expect_error("InvalidArgument", "key and value caches must have distinct storage",
                 b.causal_gqa, out, q, k, v, kc, kc, CacheLength(0), GqaSpec(2, 1, 2))
    expect_error("InvalidShape", "query heads must be a nonzero multiple of key/value heads",
                 b.causal_gqa, out, q, k, v, kc, vc, CacheLength(0), GqaSpec(3, 2, 2))


def test_conv_admission(backend):
    b = backend
    projection = up(b, np.ones((2, 12), dtype=np.float32))
    kernel = up(b, np.ones((4, 3), dtype=np.float32))
    history = up(b, np.ones((2, 4), dtype=np.float32))
    out = b.allocate_f32((2, 4))
    expect_error("InvalidArgument",
                 "short convolution hidden width and kernel width must be nonzero",
                 b.gated_short_convolution, out, projection, kernel, history,
                 GatedShortConvSpec(4, 0))
    expect_error("InvalidShape", "short convolution history must be [width - 1, hidden]",
                 b.gated_short_convolution, out, projection, up(b, np.ones((4, 2), np.float32)),
                 history, GatedShortConvSpec(4, 2))
    expect_error("InvalidShape", "short convolution projection must be [tokens, 3 * hidden]",
                 b.gated_short_convolution, out, projection, kernel, history,
                 GatedShortConvSpec(5, 3))
