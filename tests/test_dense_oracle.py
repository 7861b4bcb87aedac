"""Pins the dense oracle (oracle/mf_dense_oracle.c) before any GPU result is
compared with it: the reference's fixture cases, its strict-bit rounding
sentinels, and closed forms chosen so that a plausible slip (a wrong tap
order, head mapping, divisor or sign) fails."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from dense_fixtures import (close, conv_operands, f32, gqa_operands, head_rms_operands,
                            inference_operands, inference_ops_cases, model_ops_cases,
                            rotary_operands, sentinels)


# ---- the reference's fixtures ----------------------------------------------

@pytest.mark.parametrize("case", model_ops_cases("gated_short_convolution"), ids=lambda c: c["id"])
def test_conv_fixture(case):
    projection, kernel, history, hidden, width, expected, tail = conv_operands(case)
    out, new_history = oracle.gated_short_convolution(projection, kernel, history, hidden, width)
    assert close(out, expected)
    flat = new_history.reshape(-1)
    assert close(flat[flat.size - tail.size:], tail)


@pytest.mark.parametrize("case", model_ops_cases("split_half_rotary"), ids=lambda c: c["id"])
def test_rotary_fixture(case):
    x, positions, heads, dim, theta, expected = rotary_operands(case)
    assert close(oracle.split_half_rotary(x, positions, heads, dim, theta), expected)


def test_rotary_fixture_intermediates():
    # The fixture records the f32 frequency/angle/trig boundaries; the
    # oracle's coefficients must equal them bit for bit.
    for case in model_ops_cases("split_half_rotary"):
        x, positions, heads, dim, theta, _ = rotary_operands(case)
        half = dim // 2
        freqs = np.array([np.float32(np.float64(theta) ** (-2.0 * c / dim)) for c in range(half)],
                         dtype=np.float32)
        assert np.array_equal(freqs, f32(case["frequencies_f32"]).reshape(-1)[:half])
        angles = (positions.astype(np.float32)[:, None] * freqs[None, :]).astype(np.float32)
        assert np.array_equal(angles.reshape(-1), f32(case["angles_f32"]).reshape(-1))


@pytest.mark.parametrize("case", model_ops_cases("head_local_rms"), ids=lambda c: c["id"])
def test_head_rms_fixture(case):
    x, weight, heads, dim, eps, expected = head_rms_operands(case)
    assert close(oracle.head_rms_norm(x, weight, heads, dim, eps), expected)


@pytest.mark.parametrize("case", model_ops_cases("causal_gqa"), ids=lambda c: c["id"])
def test_gqa_fixture(case):
    o = gqa_operands(case)
    out, kc, vc, length = oracle.causal_gqa(o["query"], o["key"], o["value"], o["key_cache"],
                                            o["value_cache"], o["cache_len"], o["query_heads"],
                                            o["kv_heads"], o["head_dim"])
    assert length == o["all_keys"].shape[0]
    assert close(out, o["expected"])
    assert np.array_equal(kc, o["all_keys"]) and np.array_equal(vc, o["all_values"])


@pytest.mark.parametrize("case", inference_ops_cases(), ids=lambda c: c["id"])
def test_inference_ops_fixture(case):
    o = inference_operands(case)
    op = case["operation"]
    if op == "linear":
        got = oracle.linear(o["x"], o["weight"])
    elif op == "rms_norm":
        got = oracle.row_rms_norm(o["x"], o["weight"], np.float32(o["epsilon_f32"]))
    elif op == "embedding":
        got = oracle.gather_rows(o["weight"], np.asarray(o["token_ids"], dtype=np.int64))
    elif op == "swiglu":
        got = oracle.swiglu(o["gate"], o["up"])
    elif op == "add":
        got = oracle.add(o["left"], o["right"])
    else:
        got = oracle.multiply(o["left"], o["right"])
    assert close(got, o["expected"])


# ---- strict-bit sentinels ----------------------------------------------------

def test_rotary_sentinel_bits():
    s = sentinels()["rotary"]
    x = f32(s["input"]).reshape(1, 2)
    out = oracle.split_half_rotary(x, [s["position"]], 1, s["head_dim"], np.float32(s["theta"]))
    assert out.view(np.uint32).reshape(-1).tolist() == s["expected_u32"]
    # The f64-then-cast bits differ, so this sentinel separates the two paths.
    assert s["expected_u32"] != s["old_f64_then_cast_u32"]


def test_conv_sentinel_bits():
    s = sentinels()["convolution"]
    projection = np.concatenate([f32(s["B"]), f32(s["C"]), f32(s["V"])], axis=1)
    kernel = f32(s["kernel"])
    history = f32(s["prefix_U"])
    out, _ = oracle.gated_short_convolution(projection, kernel, history, 1, kernel.shape[1])
    assert out.view(np.uint32).reshape(-1).tolist() == np.asarray(
        s["expected_u32"]).reshape(-1).tolist()


# ---- closed forms -------------------------------------------------------------

def test_rotary_position_zero_is_identity():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((3, 4 * 8)) + 3.0).astype(np.float32)
    out = oracle.split_half_rotary(x, [0, 0, 0], 4, 8, np.float32(1e6))
    assert np.array_equal(out, x)


def test_rotary_quarter_turn_swaps_halves():
    # theta^0 = 1 for column 0, so position p rotates column 0 by p radians;
    # the oracle must produce (first cos - second sin, second cos + first sin)
    # with the trig evaluated in f64 and rounded to f32.
    x = np.array([[2.0, 3.0]], dtype=np.float32)
    out = oracle.split_half_rotary(x, [1], 1, 2, np.float32(10000.0))
    c, s = np.float32(np.cos(1.0)), np.float32(np.sin(1.0))
    assert out[0, 0] == np.float32(np.float32(2.0) * c - np.float32(3.0) * s)
    assert out[0, 1] == np.float32(np.float32(3.0) * c + np.float32(2.0) * s)


def test_rms_constant_row_closed_form():
    # Rows of 1.0 with eps 1: 1 / sqrt(4/4 + 1) = 1/sqrt(2); the mean, not the
    # sum, and eps inside the root.
    x = np.ones((2, 4), dtype=np.float32)
    w = np.array([1, 2, 3, 4], dtype=np.float32)
    out = oracle.row_rms_norm(x, w, np.float32(1.0))
    assert np.allclose(out, w[None, :] / np.sqrt(2.0), rtol=1e-7, atol=0)


def test_head_rms_is_head_local():
    # Two heads with very different scales normalise independently.
    x = np.concatenate([np.full((1, 4), 0.001), np.full((1, 4), 1000.0)], axis=1).astype(np.float32)
    out = oracle.head_rms_norm(x, np.ones(4, dtype=np.float32), 2, 4, np.float32(1e-12))
    assert np.allclose(out, 1.0, rtol=1e-5)


def test_gqa_single_key_returns_value_exactly():
    rng = np.random.default_rng(2)
    qh, kvh, d = 6, 2, 8
    q = rng.standard_normal((1, qh * d)).astype(np.float32)
    k = rng.standard_normal((1, kvh * d)).astype(np.float32)
    v = rng.standard_normal((1, kvh * d)).astype(np.float32)
    cache = np.zeros((4, kvh * d), dtype=np.float32)
    out, _, _, length = oracle.causal_gqa(q, k, v, cache, cache, 0, qh, kvh, d)
    assert length == 1
    # Query heads 0..2 read kv head 0, heads 3..5 kv head 1 (contiguous groups).
    for h in range(qh):
        kv = h // (qh // kvh)
        assert np.array_equal(out[0, h * d:(h + 1) * d], v[0, kv * d:(kv + 1) * d])


def test_gqa_matches_f64_softmax():
    rng = np.random.default_rng(3)
    qh, kvh, d, start, tokens, cap = 4, 2, 16, 5, 3, 10
    q = rng.standard_normal((tokens, qh * d)).astype(np.float32)
    k = rng.standard_normal((tokens, kvh * d)).astype(np.float32)
    v = rng.standard_normal((tokens, kvh * d)).astype(np.float32)
    kc = np.zeros((cap, kvh * d), dtype=np.float32)
    vc = np.zeros((cap, kvh * d), dtype=np.float32)
    kc[:start] = rng.standard_normal((start, kvh * d))
    vc[:start] = rng.standard_normal((start, kvh * d))
    out, kc2, vc2, length = oracle.causal_gqa(q, k, v, kc, vc, start, qh, kvh, d)
    assert length == start + tokens
    keys = np.concatenate([kc[:start], k]).astype(np.float64)
    values = np.concatenate([vc[:start], v]).astype(np.float64)
    for t in range(tokens):
        visible = start + t + 1
        for h in range(qh):
            kv = h // (qh // kvh)
            qv = q[t, h * d:(h + 1) * d].astype(np.float64)
            scores = keys[:visible, kv * d:(kv + 1) * d] @ qv / np.sqrt(d)
            p = np.exp(scores - scores.max())
            p /= p.sum()
            want = p @ values[:visible, kv * d:(kv + 1) * d]
            assert close(out[t, h * d:(h + 1) * d], want, atol=1e-5, rtol=1e-5)
    assert np.array_equal(kc2[start:start + tokens], k)
    assert np.array_equal(vc2[start:start + tokens], v)
    assert np.array_equal(kc2[:start], kc[:start])


@pytest.mark.parametrize("tap", [0, 1, 2])
@pytest.mark.parametrize("tokens", [1, 2, 5])
def test_conv_one_hot_kernel_selects_u(tap, tokens):
    rng = np.random.default_rng(4 + tap + tokens)
    hidden, width = 5, 3
    projection = rng.standard_normal((tokens, 3 * hidden)).astype(np.float32)
    history = rng.standard_normal((width - 1, hidden)).astype(np.float32)
    kernel = np.zeros((hidden, width), dtype=np.float32)
    kernel[:, tap] = 1.0
    out, new_history = oracle.gated_short_convolution(projection, kernel, history, hidden, width)
    b, c, v = (projection[:, i * hidden:(i + 1) * hidden] for i in range(3))
    u = np.concatenate([history, b * v])        # logical rows -2, -1, 0, ...
    for t in range(tokens):
        assert np.array_equal(out[t], u[t + tap] * c[t])
    assert np.array_equal(new_history, u[-(width - 1):])


def test_argmax_brute_force():
    rng = np.random.default_rng(5)
    x = rng.integers(-3, 4, size=(40, 37)).astype(np.float32)  # many ties
    got = oracle.argmax(x)
    assert np.array_equal(got, np.argmax(x, axis=1).astype(np.float32))
    x[3, 7] = np.nan
    x[9, 0] = np.inf
    got = oracle.argmax(x)
    assert np.isnan(got[3]) and np.isnan(got[9])


def test_argmax_masked_brute_force():
    rng = np.random.default_rng(6)
    x = rng.integers(-3, 4, size=(20, 130)).astype(np.float32)
    allowed = rng.random((130,)) < 0.3
    words = np.zeros(3, dtype=np.uint64)
    for i in np.nonzero(allowed)[0]:
        words[i // 64] |= np.uint64(1) << np.uint64(i % 64)
    x[0, ~allowed] = np.nan          # masked-out NaN does not poison
    got = oracle.argmax(x, words)
    masked = np.where(allowed[None, :], x, -np.inf)
    assert np.array_equal(got, np.argmax(masked, axis=1).astype(np.float32))
    assert np.all(np.isnan(oracle.argmax(x, np.zeros(3, dtype=np.uint64))))


def test_linear_matches_f64():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((5, 300)).astype(np.float32)
    w = rng.standard_normal((7, 300)).astype(np.float32)
    assert close(oracle.linear(x, w), x.astype(np.float64) @ w.astype(np.float64).T,
                 atol=1e-4, rtol=1e-4)


def test_oracle_reports_nonfinite_like_the_reference():
    x = np.array([[1e30, 1e30]], dtype=np.float32)
    with pytest.raises(oracle.OracleError) as info:
        oracle.multiply(x, x)
    assert info.value.variant == "BackendFailure"


# ---- the score-cached attention (used by the model oracle) -------------------

@pytest.mark.parametrize("tokens,start,qh,kvh,d", [(1, 0, 2, 1, 4), (5, 3, 4, 2, 8),
                                                   (17, 40, 6, 3, 16), (33, 0, 8, 8, 64)])
@pytest.mark.parametrize("threads", [1, 3, 8])
def test_cached_gqa_equals_the_literal_restatement(tokens, start, qh, kvh, d, threads):
    """The cached form keeps every sum in the reference's order over the same
    values, so it must equal the three-pass restatement bit for bit."""
    rng = np.random.default_rng(tokens * 131 + start)
    cap = start + tokens + 3
    q = rng.standard_normal((tokens, qh * d)).astype(np.float32)
    k = rng.standard_normal((tokens, kvh * d)).astype(np.float32)
    v = rng.standard_normal((tokens, kvh * d)).astype(np.float32)
    kc = np.zeros((cap, kvh * d), np.float32)
    vc = np.zeros((cap, kvh * d), np.float32)
    kc[:start] = rng.standard_normal((start, kvh * d))
    vc[:start] = rng.standard_normal((start, kvh * d))
    want = oracle.causal_gqa(q, k, v, kc, vc, start, qh, kvh, d)
    got = oracle.causal_gqa(q, k, v, kc, vc, start, qh, kvh, d, threads=threads)
    for a, b in zip(want[:3], got[:3]):
        assert a.tobytes() == b.tobytes()
    assert want[3] == got[3] == start + tokens
    kc2, vc2 = kc.copy(), vc.copy()
    got = oracle.causal_gqa(q, k, v, kc2, vc2, start, qh, kvh, d, threads=threads, in_place=True)
    assert got[1] is kc2 and kc2.tobytes() == want[1].tobytes()
    assert vc2.tobytes() == want[2].tobytes()


def test_cached_gqa_fails_like_the_literal_restatement():
    rng = np.random.default_rng(7)
    q = rng.standard_normal((4, 16)).astype(np.float32)
    k = rng.standard_normal((4, 8)).astype(np.float32)
    v = rng.standard_normal((4, 8)).astype(np.float32)
    kc = np.zeros((6, 8), np.float32)
    vc = np.full((6, 8), 9.0, np.float32)
    for bad in ("score", "value"):
        qb, vb = q.copy(), v.copy()
        if bad == "score":
            qb[2, 3] = np.inf
        else:
            vb[1, 2] = np.nan
        for threads in (0, 4):
            kc2, vc2 = kc.copy(), vc.copy()
            with pytest.raises(oracle.OracleError) as e:
                oracle.causal_gqa(qb, k, vb, kc2, vc2, 0, 2, 1, 8, threads=threads,
                                  in_place=True)
            assert e.value.variant == "BackendFailure"
            assert np.array_equal(kc2, kc) and np.array_equal(vc2, vc)
