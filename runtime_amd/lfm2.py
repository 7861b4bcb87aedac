"""LFM2 models on the HIP backend: the Python face of include/minifield_lfm2.h.

`Lfm2Model` drives the library's restatement of the reference executor's
token pass (crates/executor-core/src/lfm2/executor/execution.rs:35-585).
`synthetic_weights` builds a random-init model of a configuration (seeded
N(0, 0.02) dense weights quantized per role by the backend's converter), the
way the measured workloads are defined.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np

from . import _ffi, convert
from .backend import F32, WEIGHT, Buffer, ExecutorError, HipBackend

CONV, ATTENTION = 0, 1

# mfl_role (include/minifield_lfm2.h).
TOKEN_EMBEDDING, EMBEDDING_NORM, OPERATOR_NORM, FFN_NORM = 0, 1, 2, 3
CONV_KERNEL, CONV_IN, CONV_OUT = 4, 5, 6
QUERY_NORM, KEY_NORM, QUERY, KEY, VALUE, OUTPUT = 7, 8, 9, 10, 11, 12
FFN_W1, FFN_W2, FFN_W3 = 13, 14, 15

# The layer order of the pinned LFM2 configurations
# (crates/executor-core/tests/fixtures/pinned-lfm2.5-350m/config.json:25-42).
LFM2_LAYERS = [CONV, CONV, ATTENTION, CONV, CONV, ATTENTION, CONV, CONV, ATTENTION, CONV,
               ATTENTION, CONV, ATTENTION, CONV, ATTENTION, CONV]


@dataclass
class Lfm2Config:
    hidden: int
    intermediate: int
    attention_heads: int
    key_value_heads: int
    vocab: int
    layers: Sequence[int]
    conv_width: int = 3
    rope_theta: float = 1.0e6
    norm_epsilon: float = 1.0e-5
    block_norm_epsilon: float = 1.0e-5
    max_tokens: int = 4096
    # Stored format per matmul role: "embedding" (also the tied head),
    # "conv" (in/out), "attention" (q/k/v/o), "ffn" (w1/w2/w3); None = dense f32.
    formats: dict = field(default_factory=dict)

    @property
    def head_dim(self) -> int:
        return self.hidden // self.attention_heads

    @property
    def kv_width(self) -> int:
        return self.key_value_heads * self.head_dim


def lfm2_350m(max_tokens: int = 512) -> Lfm2Config:
    """The 350M shape, all matrices ternary: hidden 1024, FFN 4608, 16 / 8
    heads of 64, vocab 65536, tied embeddings."""
    return Lfm2Config(hidden=1024, intermediate=4608, attention_heads=16, key_value_heads=8,
                      vocab=65536, layers=list(LFM2_LAYERS), max_tokens=max_tokens,
                      formats={"embedding": "ternary", "conv": "ternary",
                               "attention": "ternary", "ffn": "ternary"})


def lfm2_1_2b(max_tokens: int = 2688) -> Lfm2Config:
    """The 1.2B shape with mixed formats: NF4 attention/conv projections,
    ternary FFN, INT8 embedding (gather and tied head)."""
    return Lfm2Config(hidden=2048, intermediate=8192, attention_heads=32, key_value_heads=8,
                      vocab=65536, layers=list(LFM2_LAYERS), max_tokens=max_tokens,
                      formats={"embedding": "int8", "conv": "nf4", "attention": "nf4",
                               "ffn": "ternary"})


def _role_group(role: int) -> str:
    if role == TOKEN_EMBEDDING:
        return "embedding"
    if role in (CONV_IN, CONV_OUT):
        return "conv"
    if role in (QUERY, KEY, VALUE, OUTPUT):
        return "attention"
    return "ffn"


def role_shapes(cfg: Lfm2Config):
    """(role, layer, shape, is_matmul) for every weight of the model, in the
    reference's plan order (weights.rs:268-470)."""
    h, inter, kv = cfg.hidden, cfg.intermediate, cfg.kv_width
    out = [(TOKEN_EMBEDDING, 0, (cfg.vocab, h), True), (EMBEDDING_NORM, 0, (h,), False)]
    for i, kind in enumerate(cfg.layers):
        if kind == CONV:
            out += [(CONV_KERNEL, i, (h, cfg.conv_width), False), (CONV_IN, i, (3 * h, h), True),
                    (CONV_OUT, i, (h, h), True)]
        else:
            out += [(QUERY_NORM, i, (cfg.head_dim,), False), (KEY_NORM, i, (cfg.head_dim,), False),
                    (QUERY, i, (h, h), True), (KEY, i, (kv, h), True), (VALUE, i, (kv, h), True),
                    (OUTPUT, i, (h, h), True)]
        out += [(FFN_W1, i, (inter, h), True), (FFN_W2, i, (h, inter), True),
                (FFN_W3, i, (inter, h), True), (OPERATOR_NORM, i, (h,), False),
                (FFN_NORM, i, (h,), False)]
    return out


class _View(Buffer):
    """A model-owned buffer seen from Python: never released from here."""
    __slots__ = ()

    def release(self) -> None:
        self._handle = 0


class Lfm2Model:
    def __init__(self, backend: HipBackend, cfg: Lfm2Config):
        self.backend = backend
        self.cfg = cfg
        kinds = (ctypes.c_uint8 * len(cfg.layers))(*cfg.layers)
        self._kinds = kinds
        c = _ffi.MflConfig(cfg.hidden, cfg.intermediate, cfg.attention_heads,
                           cfg.key_value_heads, cfg.head_dim, cfg.conv_width, cfg.vocab,
                           len(cfg.layers), ctypes.cast(kinds, ctypes.POINTER(ctypes.c_uint8)),
                           cfg.rope_theta, cfg.norm_epsilon, cfg.block_norm_epsilon,
                           cfg.max_tokens)
        out = ctypes.c_void_p()
        backend._check(_ffi.lib().mfl_create(backend.ctx, ctypes.byref(c), ctypes.byref(out)))
        self._model = out.value
        self._weights = []  # keeps attached buffers alive
        lib = _ffi.lib()
        self.logits = _View(lib.mfl_logits(self._model), backend, F32, (1, cfg.vocab))
        self.sampled = _View(lib.mfl_sampled(self._model), backend, F32, (1,))

    def close(self) -> None:
        if getattr(self, "_model", None):
            _ffi.lib().mfl_destroy(self._model)
            self._model = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_weight(self, role: int, layer: int, tensor: Buffer, scales: Buffer | None = None):
        self.backend._check(_ffi.lib().mfl_set_weight(
            self._model, role, layer, tensor.handle, scales.handle if scales else None))
        self._weights.append((tensor, scales))

    def reset(self) -> None:
        self.backend._check(_ffi.lib().mfl_reset(self._model))

    @property
    def length(self) -> int:
        return int(_ffi.lib().mfl_length(self._model))

    def append(self, tokens, produce_logits: bool = True) -> None:
        """`tokens`: host ids, or a rank-1 f32 device Buffer of ids."""
        lib = _ffi.lib()
        if isinstance(tokens, Buffer):
            status = lib.mfl_append(self._model, None, 0, tokens.handle, int(produce_logits))
        else:
            ids = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
            status = lib.mfl_append(self._model, ids.ctypes.data_as(_ffi.c_u32_p), ids.size,
                                    None, int(produce_logits))
        self.backend._check(status)

    def sample(self) -> None:
        self.backend._check(_ffi.lib().mfl_sample(self._model))

    def snapshot(self) -> "Lfm2Prefix":
        """An immutable copy of the current prefix state (mfl_snapshot)."""
        out = ctypes.c_void_p()
        self.backend._check(_ffi.lib().mfl_snapshot(self._model, ctypes.byref(out)))
        return Lfm2Prefix(out.value, self)

    def restore(self, prefix: "Lfm2Prefix") -> None:
        """Continue from `prefix` (mfl_restore); the prefix stays unchanged."""
        self.backend._check(_ffi.lib().mfl_restore(self._model, prefix.handle))

    def generate(self, steps: int, ids: Buffer | None = None) -> Buffer:
        """Greedy decode: returns the f32 device buffer of the `steps` ids."""
        ids = ids if ids is not None else self.backend.allocate_f32((steps,))
        self.backend._check(_ffi.lib().mfl_generate(self._model, steps, ids.handle))
        return ids


class Lfm2Prefix:
    """A stored prefix of one model (include/minifield_lfm2.h mfl_prefix)."""

    def __init__(self, handle: int, model: Lfm2Model):
        self._handle = handle
        self._model = model  # keeps the model (and its context) alive

    @property
    def handle(self) -> int:
        return self._handle

    @property
    def length(self) -> int:
        return int(_ffi.lib().mfl_prefix_length(self._handle))

    def close(self) -> None:
        if self._handle:
            _ffi.lib().mfl_prefix_destroy(self._handle)
            self._handle = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def synthetic_host_weights(cfg: Lfm2Config, seed: int = 0x5EED_1F00, norms: str = "ones",
                           roles=None):
    """Yield (role, layer, host arrays) of a random-init model: every matrix
    N(0, 0.02) from the counter generator (seed + 4096 * role + layer),
    quantized to its role's format as (codes, f32 scales), dense roles as
    (values,); norm weights are ones (`norms="ones"`) or 1 + N(0, 0.1)
    (`"random"`).  `roles`, when given, limits the output to those
    (role, layer) pairs."""
    for role, layer, shape, matmul in role_shapes(cfg):
        if roles is not None and (role, layer) not in roles:
            continue
        role_seed = seed + 4096 * role + layer
        if not matmul and role != CONV_KERNEL:
            if norms == "ones":
                values = np.ones(shape, dtype=np.float32)
            else:
                values = convert.normal(shape, role_seed, sigma=0.1, mean=1.0)
            yield role, layer, (values,)
            continue
        dense = convert.normal(shape, role_seed, sigma=0.02)
        fmt = cfg.formats.get(_role_group(role)) if matmul else None
        if fmt is None:
            yield role, layer, (dense,)
            continue
        codes, scales16 = convert.quantize(dense, fmt)
        del dense
        yield role, layer, (codes, convert.f16_to_f32(scales16))


def attach(model: Lfm2Model, role: int, layer: int, arrays) -> None:
    """Upload one role's host arrays (Weight class) and attach them."""
    backend = model.backend
    if len(arrays) == 2:
        codes, scales = arrays
        model.set_weight(role, layer, backend.upload_u8_classified(codes.shape, codes, WEIGHT),
                         backend.upload_f32_classified(scales.shape, scales, WEIGHT))
    else:
        (values,) = arrays
        model.set_weight(role, layer,
                         backend.upload_f32_classified(values.shape, values, WEIGHT))


def synthetic_weights(model: Lfm2Model, seed: int = 0x5EED_1F00, norms: str = "ones",
                      keep_host: bool = False):
    """Attach the random-init model of synthetic_host_weights.  Returns
    {(role, layer): host arrays} when `keep_host`."""
    host = {}
    for role, layer, arrays in synthetic_host_weights(model.cfg, seed, norms):
        attach(model, role, layer, arrays)
        if keep_host:
            host[(role, layer)] = arrays
    return host


__all__ = ["Lfm2Config", "Lfm2Model", "lfm2_350m", "lfm2_1_2b", "synthetic_weights",
           "synthetic_host_weights", "attach",
           "role_shapes", "ExecutorError", "CONV", "ATTENTION"]
