"""Loaders for the reference's dense-operator fixtures (data only).

tests/golden/model-ops-001 and tests/golden/inference-ops-001 are the
reference's NumPy-f64 operator oracles (crates/backend-cpu/tests/fixtures),
tests/golden/cr02a-rounding-sentinels-001 its strict-bit sentinels.  The
arrangement of each case into operation operands follows the reference's
own drivers (crates/backend-cpu/tests/model_ops_fixture.rs:125-340,
inference_ops_fixture.rs); JSON numbers parse as f64 and are cast to f32,
as those drivers do.
"""
from __future__ import annotations

import json
import pathlib

import numpy as np

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
# model_ops_fixture.rs:13-14 and the inference-ops manifest's tolerance rule.
ATOL, RTOL = 2.0e-6, 3.0e-5


def f32(value) -> np.ndarray:
    return np.asarray(value, dtype=np.float64).astype(np.float32)


def close(actual, expected, atol=ATOL, rtol=RTOL) -> bool:
    """|actual - expected| <= atol + rtol * |expected| on every element, all
    finite (model_ops_fixture.rs `close`)."""
    a = np.asarray(actual, dtype=np.float64).reshape(-1)
    e = np.asarray(expected, dtype=np.float64).reshape(-1)
    if a.shape != e.shape or not np.all(np.isfinite(a)):
        return False
    return bool(np.all(np.abs(a - e) <= atol + rtol * np.abs(e)))


def _load(name):
    return json.loads((GOLDEN / name / "cases.json").read_text())


def model_ops_cases(operation: str | None = None):
    cases = _load("model-ops-001")["cases"]
    return [c for c in cases if operation is None or c["operation"] == operation]


def inference_ops_cases(operation: str | None = None):
    cases = _load("inference-ops-001")["cases"]
    return [c for c in cases if operation is None or c["operation"] == operation]


def sentinels():
    return json.loads((GOLDEN / "cr02a-rounding-sentinels-001" / "rounding-sentinels.json")
                      .read_text())


def conv_operands(case):
    """(projection [T, 3h], kernel [h, w], history [w-1, h], hidden, width,
    expected output [T, h], expected history tail)."""
    b, c, v = f32(case["B"]), f32(case["C"]), f32(case["V"])
    kernel = f32(case["kernel"])
    tokens, hidden = b.shape
    width = kernel.shape[1]
    projection = np.concatenate([b, c, v], axis=1)
    history = np.zeros(((width - 1), hidden), dtype=np.float32)
    prefix = f32(case["prefix_U"]).reshape(-1)
    if prefix.size:
        history.reshape(-1)[history.size - prefix.size:] = prefix
    tail = f32(case["tail_U"]).reshape(-1)
    return projection, kernel, history, hidden, width, f32(case["output"]), tail


def rotary_operands(case):
    """(input [T, heads * dim], positions, heads, dim, theta, expected)."""
    x = f32(case["input"])
    tokens, heads, dim = x.shape
    positions = np.asarray(case["positions"], dtype=np.uint64)
    return (x.reshape(tokens, heads * dim), positions, heads, dim, np.float32(case["theta"]),
            f32(case["output"]).reshape(tokens, heads * dim))


def head_rms_operands(case):
    """(input [T, heads * dim], weight [dim], heads, dim, epsilon, expected)."""
    x = f32(case["input"])
    tokens, heads, dim = x.shape
    return (x.reshape(tokens, heads * dim), f32(case["weight"]), heads, dim,
            np.float32(case["epsilon"]), f32(case["output"]).reshape(tokens, heads * dim))


def gqa_operands(case):
    """Operands as model_ops_fixture.rs:268-322 arranges them: the query
    rows from `query_start`, the key/value tails as the new rows, caches of
    capacity `total` prefilled with the first `query_start` rows."""
    q, k, v = f32(case["Q"]), f32(case["K"]), f32(case["V"])
    tokens, query_heads, dim = q.shape
    total, kv_heads, _ = k.shape
    start = int(case["query_start"])
    kv_width = kv_heads * dim
    keys = k.reshape(total, kv_width)
    values = v.reshape(total, kv_width)
    key_cache = np.zeros((total, kv_width), dtype=np.float32)
    value_cache = np.zeros((total, kv_width), dtype=np.float32)
    key_cache[:start] = keys[:start]
    value_cache[:start] = values[:start]
    return dict(query=q.reshape(tokens, query_heads * dim), key=keys[start:].copy(),
                value=values[start:].copy(), key_cache=key_cache, value_cache=value_cache,
                cache_len=start, query_heads=query_heads, kv_heads=kv_heads, head_dim=dim,
                expected=f32(case["output"]).reshape(tokens, query_heads * dim),
                all_keys=keys, all_values=values)


def inference_operands(case):
    """name -> f32 array (shaped) for an inference-ops-001 case's inputs,
    plus `expected`."""
    out = {}
    for name, spec in case["inputs"].items():
        if isinstance(spec, dict) and "f32_values" in spec:
            out[name] = f32(spec["f32_values"]).reshape(spec["shape"])
        else:
            out[name] = spec
    exp = case["expected"]
    out["expected"] = f32(exp["f32_values"]).reshape(exp["shape"])
    return out
