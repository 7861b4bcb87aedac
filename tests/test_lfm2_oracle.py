"""Pins the LFM2 pass oracle (oracle/lfm2_model.py) on the CPU.

1. An independent float64 numpy forward over dequantized weights: written
   from the model definition (pre-norm blocks, B*V gated short convolution,
   GQA with per-head q/k RMS and split-half RoPE, SwiGLU FFN, tied head), not
   from the executor's call sequence, so a wrong residual wiring, norm
   placement, head mapping or position would disagree far beyond the
   rounding gap between f32 and f64.
2. Prefill equals token-by-token appends bitwise (caches, history and
   positions carry state exactly).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle.lfm2_model import OracleLfm2
from runtime_amd import convert
from runtime_amd.lfm2 import (ATTENTION, CONV, CONV_IN, CONV_KERNEL, CONV_OUT, EMBEDDING_NORM,
                              FFN_NORM, FFN_W1, FFN_W2, FFN_W3, KEY, KEY_NORM, OPERATOR_NORM,
                              OUTPUT, QUERY, QUERY_NORM, TOKEN_EMBEDDING, VALUE, Lfm2Config,
                              role_shapes)

FORMATS = {"embedding": "int8", "conv": "nf4", "attention": "ternary", "ffn": "nf4"}


def tiny(formats=FORMATS):
    return Lfm2Config(hidden=128, intermediate=256, attention_heads=4, key_value_heads=2,
                      vocab=300, layers=[CONV, ATTENTION, CONV, ATTENTION], max_tokens=64,
                      formats=dict(formats))


def host_weights(cfg, seed=0x51):
    """The same recipe as runtime_amd.lfm2.synthetic_weights, on the host."""
    groups = {TOKEN_EMBEDDING: "embedding", CONV_IN: "conv", CONV_OUT: "conv",
              QUERY: "attention", KEY: "attention", VALUE: "attention", OUTPUT: "attention"}
    out = {}
    for role, layer, shape, matmul in role_shapes(cfg):
        s = seed + 4096 * role + layer
        if not matmul and role != CONV_KERNEL:
            out[(role, layer)] = (convert.normal(shape, s, sigma=0.1, mean=1.0),)
            continue
        dense = convert.normal(shape, s, sigma=0.02 if matmul else 0.3)
        fmt = cfg.formats.get(groups.get(role, "ffn")) if matmul else None
        if fmt is None:
            out[(role, layer)] = (dense,)
        else:
            codes, scales16 = convert.quantize(dense, fmt)
            out[(role, layer)] = (codes, convert.f16_to_f32(scales16), fmt)
    return out


def dense_of(entry):
    if len(entry) == 1:
        return entry[0].astype(np.float64)
    codes, scales, fmt = entry
    return oracle.dequantize_f32(codes, scales, fmt).astype(np.float64)


def f64_forward(cfg, w, tokens):
    """Float64 LFM2 forward over all tokens; returns the last row's logits."""
    h, d, qh, kvh = cfg.hidden, cfg.head_dim, cfg.attention_heads, cfg.key_value_heads
    W = {k: dense_of(v) for k, v in w.items()}
    T = len(tokens)

    def rms(x, g, eps):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * g

    def rope(x, pos):  # x [T, heads, d]
        half = d // 2
        freq = cfg.rope_theta ** (-2.0 * np.arange(half) / d)
        ang = pos[:, None] * freq[None, :]
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        a, b = x[..., :half], x[..., half:]
        return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)

    x = W[(TOKEN_EMBEDDING, 0)][np.asarray(tokens)]
    pos = np.arange(T, dtype=np.float64)
    for i, kind in enumerate(cfg.layers):
        u = rms(x, W[(OPERATOR_NORM, i)], cfg.block_norm_epsilon)
        if kind == CONV:
            p = u @ W[(CONV_IN, i)].T
            b, c, v = p[:, :h], p[:, h:2 * h], p[:, 2 * h:]
            bv = np.concatenate([np.zeros((cfg.conv_width - 1, h)), b * v])
            k = W[(CONV_KERNEL, i)]  # [h, width], oldest to current
            conv = sum(k[:, j] * bv[j:j + T] for j in range(cfg.conv_width))
            op = (conv * c) @ W[(CONV_OUT, i)].T
        else:
            q = (u @ W[(QUERY, i)].T).reshape(T, qh, d)
            kk = (u @ W[(KEY, i)].T).reshape(T, kvh, d)
            vv = (u @ W[(VALUE, i)].T).reshape(T, kvh, d)
            q = rope(rms(q, W[(QUERY_NORM, i)], cfg.block_norm_epsilon), pos)
            kk = rope(rms(kk, W[(KEY_NORM, i)], cfg.block_norm_epsilon), pos)
            att = np.zeros((T, qh, d))
            for head in range(qh):
                g = head // (qh // kvh)
                scores = q[:, head] @ kk[:, g].T / np.sqrt(d)
                scores[np.triu_indices(T, 1)] = -np.inf
                p_ = np.exp(scores - scores.max(axis=1, keepdims=True))
                p_ /= p_.sum(axis=1, keepdims=True)
                att[:, head] = p_ @ vv[:, g]
            op = att.reshape(T, h) @ W[(OUTPUT, i)].T
        x = x + op
        f = rms(x, W[(FFN_NORM, i)], cfg.block_norm_epsilon)
        g1, g3 = f @ W[(FFN_W1, i)].T, f @ W[(FFN_W3, i)].T
        x = x + ((g1 / (1 + np.exp(-g1))) * g3) @ W[(FFN_W2, i)].T
    u = rms(x[-1:], W[(EMBEDDING_NORM, 0)], cfg.norm_epsilon)
    return u @ W[(TOKEN_EMBEDDING, 0)].T


def oracle_weights(w):
    return {k: v[:2] if len(v) == 3 else v for k, v in w.items()}


@pytest.mark.parametrize("tokens", [1, 5, 12])
def test_oracle_pass_matches_f64_model(tokens):
    cfg = tiny()
    w = host_weights(cfg)
    ids = convert.token_ids(tokens, 0x7043_0010 + tokens, cfg.vocab)
    got = OracleLfm2(cfg, oracle_weights(w)).append(ids)
    want = f64_forward(cfg, w, ids)
    err = np.max(np.abs(got - want)) / np.max(np.abs(want))
    assert err < 2e-5, err


def test_oracle_pass_dense_roles_match_f64_model():
    cfg = tiny({"embedding": None, "conv": None, "attention": None, "ffn": "int8"})
    w = host_weights(cfg, seed=0x52)
    ids = convert.token_ids(6, 0x7043_0020, cfg.vocab)
    got = OracleLfm2(cfg, oracle_weights(w)).append(ids)
    want = f64_forward(cfg, w, ids)
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 2e-5


def test_oracle_prefill_equals_stepwise_appends():
    cfg = tiny()
    w = oracle_weights(host_weights(cfg))
    ids = convert.token_ids(8, 0x7043_0030, cfg.vocab)
    whole = OracleLfm2(cfg, w).append(ids)
    stepwise = OracleLfm2(cfg, w)
    for t in ids:
        last = stepwise.append([t])
    assert np.array_equal(whole.view(np.uint32), last.view(np.uint32))
    assert stepwise.length == 8


def test_oracle_detects_a_miswired_residual():
    # A plausible slip -- the FFN reading the pre-norm residual -- must
    # exceed the tolerance the f64 comparison uses.
    cfg = tiny()
    w = host_weights(cfg)
    ids = convert.token_ids(5, 0x7043_0040, cfg.vocab)
    good = f64_forward(cfg, w, ids)
    ref = OracleLfm2(cfg, oracle_weights(w))
    original = oracle.add_row_rms_norm
    try:
        oracle.add_row_rms_norm = lambda l, r, g, e: (original(l, r, g, e)[0],
                                                      original(l, r, g, e)[0])
        bad = ref.append(ids)
    finally:
        oracle.add_row_rms_norm = original
    assert np.max(np.abs(bad - good)) / np.max(np.abs(good)) > 1e-3


def test_single_threaded_pass_equals_the_parallel_one():
    """threads=1 (the CPU baseline: every operation single-threaded, scans
    included, literal attention) gives the parallel pass's bits, prefill and
    decode, and its per-operation timings cover every operation kind."""
    cfg = tiny()
    w = oracle_weights(host_weights(cfg))
    ids = convert.token_ids(7, 0x7043_0050, cfg.vocab)
    timings = {}
    single = OracleLfm2(cfg, w, threads=1, timings=timings)
    parallel = OracleLfm2(cfg, w, threads=4)
    for model in (single, parallel):
        model.append(ids)
    assert single.logits.tobytes() == parallel.logits.tobytes()
    for _ in range(3):
        tokens = [single.sample(), parallel.sample()]
        assert tokens[0] == tokens[1]
        single.append([int(tokens[0])])
        parallel.append([int(tokens[1])])
        assert single.logits.tobytes() == parallel.logits.tobytes()
    assert {"embedding gather", "norms", "conv in projection", "short convolution",
            "conv out projection", "q/k/v projections", "qk norm + rope", "attention",
            "attention out projection", "ffn gate/up", "swiglu", "ffn down", "lm head",
            "argmax"} <= set(timings)
