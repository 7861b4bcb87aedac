"""CPU oracle of the packed-weight path -- TEST INFRASTRUCTURE ONLY.

numpy wrappers over oracle/libmf_oracle.so, the C restatement of the
reference's scalar CPU backend (see mf_oracle.c for the file:line citations).
Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use it,
always as the checker, never as the thing measured or shipped.
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess
import threading

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIBRARY_PATH = HERE / "libmf_oracle.so"

FORMATS = {"ternary": 0, "nf4": 1, "int8": 2}
WPB = {"ternary": 4, "nf4": 2, "int8": 1}
STATUS_NAMES = {0: "Ok", 1: "InvalidArgument", 2: "InvalidShape", 6: "OutOfBounds",
                8: "ResourceLimit", 17: "BackendFailure"}

_f = ctypes.POINTER(ctypes.c_float)
_u8 = ctypes.POINTER(ctypes.c_uint8)
_d = ctypes.POINTER(ctypes.c_double)
_i64 = ctypes.POINTER(ctypes.c_int64)
_u64 = ctypes.POINTER(ctypes.c_uint64)
_SZ = ctypes.c_size_t

_SIGS = {
    "mfo_ternary_row_dot": (ctypes.c_float, [_u8, _f, _f, _SZ]),
    "mfo_nf4_row_dot": (ctypes.c_float, [_u8, _f, _f, _SZ]),
    "mfo_int8_row_dot": (ctypes.c_float, [_u8, _f, _f, _SZ]),
    "mfo_packed_format": (ctypes.c_int, [_SZ, _SZ, _SZ, _u8, ctypes.POINTER(ctypes.c_int)]),
    "mfo_packed_linear": (ctypes.c_int, [_f, _f, _SZ, _u8, _f, _SZ, _SZ, _SZ]),
    "mfo_packed_linear_rows": (ctypes.c_int, [_f, _f, _SZ, _u8, _f, _SZ, _SZ, _SZ, _SZ, _SZ]),
    "mfo_packed_linear_pair": (ctypes.c_int, [_f, _f, _f, _SZ, _u8, _f, _u8, _f, _SZ, _SZ, _SZ]),
    "mfo_packed_swiglu_pair": (ctypes.c_int, [_f, _f, _SZ, _u8, _f, _u8, _f, _SZ, _SZ, _SZ]),
    "mfo_packed_swiglu_linear": (ctypes.c_int, [_f, _f, _f, _SZ, _u8, _f, _SZ, _SZ, _SZ]),
    "mfo_swiglu": (None, [_f, _f, _f, _SZ]),
    "mfo_resolve_device_ids": (None, [_f, _SZ, _i64]),
    "mfo_packed_gather_rows": (ctypes.c_int, [_f, _u8, _f, _SZ, _SZ, _SZ, _i64, _SZ]),
    "mfo_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "mfo_dense_f64": (None, [_d, _f, _SZ, _f, _SZ, _SZ]),
    "mfo_row_rms_norm": (ctypes.c_int, [_f, _f, _f, _SZ, _SZ, ctypes.c_float]),
    "mfo_head_rms_norm": (ctypes.c_int, [_f, _f, _f, _SZ, _SZ, _SZ, ctypes.c_float]),
    "mfo_split_half_rotary": (ctypes.c_int, [_f, _f, _u64, _SZ, _SZ, _SZ, ctypes.c_float]),
    "mfo_qk_norm_rope": (ctypes.c_int, [_f, _f, _f, _f, _f, _f, _u64, _SZ, _SZ, _SZ, _SZ,
                                        ctypes.c_float, ctypes.c_float]),
    "mfo_elementwise": (ctypes.c_int, [_f, _f, _f, _SZ, ctypes.c_int]),
    "mfo_linear": (ctypes.c_int, [_f, _f, _f, _SZ, _SZ, _SZ]),
    "mfo_argmax": (None, [_f, _f, _SZ, _SZ, _u64]),
    "mfo_gather_rows": (ctypes.c_int, [_f, _f, _SZ, _SZ, _i64, _SZ]),
    "mfo_causal_gqa": (ctypes.c_int, [_f, _f, _f, _f, _f, _f, _u64, _SZ, _SZ, _SZ, _SZ]),
    "mfo_causal_gqa_cached": (ctypes.c_int, [_f, _f, _f, _f, _f, _f, _u64, _SZ, _SZ, _SZ, _SZ,
                                             _SZ]),
    "mfo_gated_short_convolution": (ctypes.c_int, [_f, _f, _f, _f, _SZ, _SZ, _SZ]),
}

_lib = None
_lock = threading.Lock()


class OracleError(Exception):
    def __init__(self, status: int):
        self.status = status
        self.variant = STATUS_NAMES.get(status, f"Status{status}")
        super().__init__(self.variant)


def build() -> pathlib.Path:
    """Compile the oracle with its Makefile (always rebuilds)."""
    subprocess.run(["make", "-B", "-s", "-C", str(HERE)], check=True)
    return LIBRARY_PATH


def lib():
    global _lib
    with _lock:
        if _lib is None:
            if not LIBRARY_PATH.exists():
                build()
            handle = ctypes.CDLL(str(LIBRARY_PATH))
            for name, (res, args) in _SIGS.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def _fp(a):
    return a.ctypes.data_as(_f)


def _u8p(a):
    return a.ctypes.data_as(_u8)


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _cu8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def _check(status):
    if status:
        raise OracleError(status)


def row_dot(scheme: str, codes, scales, x) -> np.float32:
    codes, scales, x = _cu8(codes), _c32(scales), _c32(x)
    fn = getattr(lib(), f"mfo_{scheme}_row_dot")
    return np.float32(fn(_u8p(codes), _fp(scales), _fp(x), x.size))


def packed_format(codes, scales) -> str:
    codes = _cu8(codes)
    fmt = ctypes.c_int(-1)
    _check(lib().mfo_packed_format(codes.shape[0], codes.shape[1], scales.shape[1],
                                   _u8p(codes), ctypes.byref(fmt)))
    return {0: "ternary", 1: "nf4", 2: "int8"}[fmt.value]


def packed_linear(x, codes, scales, out=None) -> np.ndarray:
    """CpuBackend::packed_linear (backend-cpu/src/packed.rs:96-170)."""
    x, codes, scales = _c32(x), _cu8(codes), _c32(scales)
    m, n = x.shape[0], codes.shape[0]
    out = np.zeros((m, n), dtype=np.float32) if out is None else out
    _check(lib().mfo_packed_linear(_fp(out), _fp(x), m, _u8p(codes), _fp(scales), n,
                                   codes.shape[1], scales.shape[1]))
    return out


def packed_linear_threaded(x, codes, scales, threads: int = 8) -> np.ndarray:
    """Same bits as packed_linear, output columns split across threads."""
    x, codes, scales = _c32(x), _cu8(codes), _c32(scales)
    m, n = x.shape[0], codes.shape[0]
    out = np.zeros((m, n), dtype=np.float32)
    chunk = (n + threads - 1) // threads
    fn = lib().mfo_packed_linear_rows

    def work(begin):
        _check(fn(_fp(out), _fp(x), m, _u8p(codes), _fp(scales), n, codes.shape[1],
                  scales.shape[1], begin, min(n, begin + chunk)))

    pool = [threading.Thread(target=work, args=(b,)) for b in range(0, n, chunk)]
    for t in pool:
        t.start()
    for t in pool:
        t.join()
    return out


def packed_linear_pair(x, codes_a, scales_a, codes_b, scales_b):
    x = _c32(x)
    codes_a, codes_b = _cu8(codes_a), _cu8(codes_b)
    scales_a, scales_b = _c32(scales_a), _c32(scales_b)
    m, n = x.shape[0], codes_a.shape[0]
    out_a = np.zeros((m, n), dtype=np.float32)
    out_b = np.zeros((m, n), dtype=np.float32)
    _check(lib().mfo_packed_linear_pair(_fp(out_a), _fp(out_b), _fp(x), m, _u8p(codes_a),
                                        _fp(scales_a), _u8p(codes_b), _fp(scales_b), n,
                                        codes_a.shape[1], scales_a.shape[1]))
    return out_a, out_b


def packed_swiglu_pair(x, codes_a, scales_a, codes_b, scales_b):
    x = _c32(x)
    codes_a, codes_b = _cu8(codes_a), _cu8(codes_b)
    scales_a, scales_b = _c32(scales_a), _c32(scales_b)
    m, n = x.shape[0], codes_a.shape[0]
    out = np.zeros((m, n), dtype=np.float32)
    _check(lib().mfo_packed_swiglu_pair(_fp(out), _fp(x), m, _u8p(codes_a), _fp(scales_a),
                                        _u8p(codes_b), _fp(scales_b), n, codes_a.shape[1],
                                        scales_a.shape[1]))
    return out


def packed_swiglu_linear(gate, up, codes, scales):
    gate, up, codes, scales = _c32(gate), _c32(up), _cu8(codes), _c32(scales)
    m, n = gate.shape[0], codes.shape[0]
    out = np.zeros((m, n), dtype=np.float32)
    _check(lib().mfo_packed_swiglu_linear(_fp(out), _fp(gate), _fp(up), m, _u8p(codes),
                                          _fp(scales), n, codes.shape[1], scales.shape[1]))
    return out


def swiglu(gate, up):
    gate, up = _c32(gate), _c32(up)
    out = np.empty_like(gate)
    lib().mfo_swiglu(_fp(out), _fp(gate), _fp(up), gate.size)
    return out


def resolve_device_ids(values) -> np.ndarray:
    values = _c32(values).reshape(-1)
    ids = np.empty(values.size, dtype=np.int64)
    lib().mfo_resolve_device_ids(_fp(values), values.size, ids.ctypes.data_as(_i64))
    return ids


def packed_gather_rows(codes, scales, ids) -> np.ndarray:
    """ids: int64 row ids, -1 for a None (NaN) row."""
    codes, scales = _cu8(codes), _c32(scales)
    ids = np.ascontiguousarray(ids, dtype=np.int64).reshape(-1)
    inner = scales.shape[1] * 128
    out = np.zeros((ids.size, inner), dtype=np.float32)
    _check(lib().mfo_packed_gather_rows(_fp(out), _u8p(codes), _fp(scales), codes.shape[0],
                                        codes.shape[1], scales.shape[1],
                                        ids.ctypes.data_as(_i64), ids.size))
    return out


def f16_to_f32(bits: int) -> np.float32:
    return np.float32(lib().mfo_f16_to_f32(bits))


def dense_f64(x, weights) -> np.ndarray:
    x, weights = _c32(x), _c32(weights)
    m, k = x.shape
    n = weights.shape[0]
    out = np.zeros((m, n), dtype=np.float64)
    lib().mfo_dense_f64(out.ctypes.data_as(_d), _fp(x), m, _fp(weights), n, k)
    return out


NF4_LEVELS = np.array([
    -1.0, -0.6961928, -0.52507305, -0.3949175, -0.28444138, -0.18477343, -0.091050036, 0.0,
    0.0795803, 0.1609302, 0.2461123, 0.33791524, 0.44070983, 0.562617, 0.72295684, 1.0,
], dtype=np.float32)


def dequantize_f32(codes, scales, scheme: str) -> np.ndarray:
    """Dequantize canonical codes with f32 scales (w = level * scale, one f32
    multiply, as packed_gather_rows does), vectorised in numpy."""
    codes, scales = _cu8(codes), _c32(scales)
    rows = codes.shape[0]
    if scheme == "ternary":
        q = np.stack([(codes >> (2 * j)) & 3 for j in range(4)], axis=-1).reshape(rows, -1)
        levels = q.astype(np.float32) - np.float32(1)
    elif scheme == "nf4":
        q = np.stack([codes & 15, codes >> 4], axis=-1).reshape(rows, -1)
        levels = NF4_LEVELS[q]
    else:
        levels = codes.view(np.int8).astype(np.float32)
    return levels * np.repeat(scales, 128, axis=1)


# ---- dense LFM2 operations (mf_dense_oracle.c) -----------------------------

def _cu64(a):
    return np.ascontiguousarray(a, dtype=np.uint64).reshape(-1)


def row_rms_norm(x, weight, epsilon) -> np.ndarray:
    """CpuBackend::row_rms_norm over [rows, width]."""
    x, weight = _c32(x), _c32(weight)
    out = np.zeros_like(x)
    _check(lib().mfo_row_rms_norm(_fp(out), _fp(x), _fp(weight), x.shape[0], x.shape[1],
                                  epsilon))
    return out


def head_rms_norm(x, weight, heads, head_dim, epsilon) -> np.ndarray:
    x, weight = _c32(x), _c32(weight)
    out = np.zeros_like(x)
    _check(lib().mfo_head_rms_norm(_fp(out), _fp(x), _fp(weight), x.shape[0], heads, head_dim,
                                   epsilon))
    return out


def split_half_rotary(x, positions, heads, head_dim, theta) -> np.ndarray:
    x, pos = _c32(x), _cu64(positions)
    out = np.zeros_like(x)
    _check(lib().mfo_split_half_rotary(_fp(out), _fp(x), pos.ctypes.data_as(_u64), x.shape[0],
                                       heads, head_dim, theta))
    return out


def qk_norm_rope(query, key, query_weight, key_weight, positions, query_heads, key_heads,
                 head_dim, theta, epsilon):
    query, key = _c32(query), _c32(key)
    qw, kw, pos = _c32(query_weight), _c32(key_weight), _cu64(positions)
    q_out, k_out = np.zeros_like(query), np.zeros_like(key)
    _check(lib().mfo_qk_norm_rope(_fp(q_out), _fp(k_out), _fp(query), _fp(key), _fp(qw),
                                  _fp(kw), pos.ctypes.data_as(_u64), query.shape[0],
                                  query_heads, key_heads, head_dim, theta, epsilon))
    return q_out, k_out


def add(left, right) -> np.ndarray:
    left, right = _c32(left), _c32(right)
    out = np.zeros_like(left)
    _check(lib().mfo_elementwise(_fp(out), _fp(left), _fp(right), left.size, 0))
    return out


def multiply(left, right) -> np.ndarray:
    left, right = _c32(left), _c32(right)
    out = np.zeros_like(left)
    _check(lib().mfo_elementwise(_fp(out), _fp(left), _fp(right), left.size, 1))
    return out


def add_row_rms_norm(left, right, weight, epsilon):
    """CpuBackend::add_row_rms_norm: add, then row_rms_norm of the sum."""
    total = add(left, right)
    return total, row_rms_norm(total, weight, epsilon)


def linear(x, weight) -> np.ndarray:
    x, weight = _c32(x), _c32(weight)
    m, k = x.shape
    n = weight.shape[0]
    out = np.zeros((m, n), dtype=np.float32)
    _check(lib().mfo_linear(_fp(out), _fp(x), _fp(weight), m, n, k))
    return out


def argmax(x, mask=None) -> np.ndarray:
    x = _c32(x)
    out = np.zeros(x.shape[0], dtype=np.float32)
    mask_ptr = None
    if mask is not None:
        mask = _cu64(mask)
        mask_ptr = mask.ctypes.data_as(_u64)
    lib().mfo_argmax(_fp(out), _fp(x), x.shape[0], x.shape[1], mask_ptr)
    return out


def gather_rows(table, ids) -> np.ndarray:
    """ids: int64 row ids, -1 for a None (NaN) row."""
    table = _c32(table)
    ids = np.ascontiguousarray(ids, dtype=np.int64).reshape(-1)
    out = np.zeros((ids.size, table.shape[1]), dtype=np.float32)
    _check(lib().mfo_gather_rows(_fp(out), _fp(table), table.shape[0], table.shape[1],
                                 ids.ctypes.data_as(_i64), ids.size))
    return out


def gather_columns(x, columns) -> np.ndarray:
    """CpuBackend::gather_columns (dense.rs:143-149): out[r, k] = x[r, columns[k]]."""
    x = _c32(x)
    return np.ascontiguousarray(x[:, np.asarray(columns, dtype=np.int64)])


def copy_rect_2d(dst, src, rect) -> np.ndarray:
    """CpuBackend::copy_rect_2d (dense.rs:311-339) on a copy of `dst`;
    rect = (source_row, source_column, destination_row, destination_column,
    rows, columns)."""
    sr, sc, dr, dc, rows, cols = rect
    out = _c32(dst).copy()
    out[dr:dr + rows, dc:dc + cols] = _c32(src)[sr:sr + rows, sc:sc + cols]
    return out


def causal_gqa(query, key, value, key_cache, value_cache, cache_len, query_heads, key_heads,
               head_dim, threads: int = 0, in_place: bool = False):
    """Returns (output, key_cache, value_cache, new_cache_len).  The caches
    passed in are not modified unless `in_place` (then they are returned,
    updated).  `threads` > 0 takes the score-cached restatement on that many
    threads (the same bits)."""
    query, key, value = _c32(query), _c32(key), _c32(value)
    if in_place:
        kc, vc = key_cache, value_cache
        assert kc.dtype == np.float32 and vc.dtype == np.float32
        assert kc.flags.c_contiguous and vc.flags.c_contiguous
    else:
        kc, vc = _c32(key_cache).copy(), _c32(value_cache).copy()
    out = np.zeros_like(query)
    length = ctypes.c_uint64(cache_len)
    args = (_fp(out), _fp(query), _fp(key), _fp(value), _fp(kc), _fp(vc), ctypes.byref(length),
            query.shape[0], query_heads, key_heads, head_dim)
    if threads > 0:
        _check(lib().mfo_causal_gqa_cached(*args, threads))
    else:
        _check(lib().mfo_causal_gqa(*args))
    return out, kc, vc, length.value


def gated_short_convolution(projection, kernel, history, hidden, width):
    """Returns (output, new_history); the history passed in is not modified."""
    projection, kernel = _c32(projection), _c32(kernel)
    hist = _c32(history).copy()
    tokens = projection.shape[0]
    out = np.zeros((tokens, hidden), dtype=np.float32)
    _check(lib().mfo_gated_short_convolution(_fp(out), _fp(projection), _fp(kernel), _fp(hist),
                                             tokens, hidden, width))
    return out, hist
