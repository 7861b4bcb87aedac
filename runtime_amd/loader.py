"""safetensors bundles on the HIP backend: the Python face of
include/minifield_loader.h.

`SafetensorsFile` opens and validates a bundle with the reference loader's
header rules (crates/executor-core/src/loader/header.rs); `upload_packed` /
`upload_dense` move one role's streams straight to device buffers (packed
scales stay binary16 on the device); `load_lfm2` attaches a whole LFM2 model
by the reference's tensor names.  `write_lfm2_bundle` writes a bundle in the
converter's layout (tools/converters/src/minifield_converters/preparation.py:
226-260): codes U8, scales F16, dense tensors F32, `minifield.mixed.v1` with a
per-tensor `tensor_quantization` map.
"""
from __future__ import annotations

import ctypes
import json

import numpy as np

from . import _ffi
from .backend import F32, U8, WEIGHT, Buffer, ExecutorError, HipBackend

DTYPES = {0: "F32", 1: "BF16", 2: "F16", 3: "U8"}
SCHEMES = {0: "dense", 1: "ternary", 2: "nf4", 3: "int8"}


def _check(status: int) -> None:
    if status:
        raise ExecutorError(status, _ffi.lib().mfs_error().decode())


class SafetensorsFile:
    def __init__(self, path, max_header_bytes: int = 0):
        out = ctypes.c_void_p()
        _check(_ffi.lib().mfs_open(str(path).encode(), max_header_bytes, ctypes.byref(out)))
        self._handle = out.value

    @property
    def handle(self) -> int:
        return self._handle

    def close(self) -> None:
        if getattr(self, "_handle", None):
            _ffi.lib().mfs_close(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def names(self) -> list[str]:
        lib = _ffi.lib()
        return [lib.mfs_tensor_name(self._handle, i).decode()
                for i in range(lib.mfs_tensor_count(self._handle))]

    def info(self, name: str):
        """(dtype name, shape) of a tensor."""
        dtype = ctypes.c_int(0)
        rank = ctypes.c_uint32(0)
        dims = (ctypes.c_uint64 * 4)()
        _check(_ffi.lib().mfs_tensor_info(self._handle, name.encode(), ctypes.byref(dtype),
                                          ctypes.byref(rank), dims))
        return DTYPES[dtype.value], tuple(int(dims[i]) for i in range(rank.value))

    def metadata(self, key: str) -> str | None:
        value = _ffi.lib().mfs_metadata(self._handle, key.encode())
        return None if value is None else value.decode()

    def matmul_scheme(self, name: str) -> str:
        out = ctypes.c_int(0)
        _check(_ffi.lib().mfs_matmul_scheme(self._handle, name.encode(), ctypes.byref(out)))
        return SCHEMES[out.value]

    def upload_packed(self, backend: HipBackend, base: str, cls: int = WEIGHT):
        codes, scales = ctypes.c_void_p(), ctypes.c_void_p()
        status = _ffi.lib().mfs_upload_packed(backend.ctx, self._handle, base.encode(), cls,
                                              ctypes.byref(codes), ctypes.byref(scales))
        _check(status)
        _, cshape = self.info(base + ".codes")
        _, sshape = self.info(base + ".scales")
        return Buffer(codes.value, backend, U8, cshape), Buffer(scales.value, backend, F32, sshape)

    def upload_dense(self, backend: HipBackend, name: str, cls: int = WEIGHT) -> Buffer:
        out = ctypes.c_void_p()
        _check(_ffi.lib().mfs_upload_dense(backend.ctx, self._handle, name.encode(), cls,
                                           ctypes.byref(out)))
        return Buffer(out.value, backend, F32, self.info(name)[1])


def load_lfm2(model, bundle: SafetensorsFile) -> None:
    """Attach every role of `model` (an Lfm2Model) from `bundle`."""
    status = _ffi.lib().mfl_load_safetensors(model._model, bundle.handle)
    if status:
        raise ExecutorError(status, model.backend.last_error())


def lfm2_tensor_names(cfg):
    """{(role, layer): tensor name} of the reference's LFM2 plan
    (crates/executor-core/src/lfm2/weights.rs:268-500)."""
    from . import lfm2 as L
    names = {(L.TOKEN_EMBEDDING, 0): "model.embed_tokens.weight",
             (L.EMBEDDING_NORM, 0): "model.embedding_norm.weight"}
    for i, kind in enumerate(cfg.layers):
        p = f"model.layers.{i}"
        if kind == L.CONV:
            names[(L.CONV_KERNEL, i)] = f"{p}.conv.conv.weight"
            names[(L.CONV_IN, i)] = f"{p}.conv.in_proj.weight"
            names[(L.CONV_OUT, i)] = f"{p}.conv.out_proj.weight"
        else:
            names[(L.QUERY_NORM, i)] = f"{p}.self_attn.q_layernorm.weight"
            names[(L.KEY_NORM, i)] = f"{p}.self_attn.k_layernorm.weight"
            names[(L.QUERY, i)] = f"{p}.self_attn.q_proj.weight"
            names[(L.KEY, i)] = f"{p}.self_attn.k_proj.weight"
            names[(L.VALUE, i)] = f"{p}.self_attn.v_proj.weight"
            names[(L.OUTPUT, i)] = f"{p}.self_attn.out_proj.weight"
        names[(L.FFN_W1, i)] = f"{p}.feed_forward.w1.weight"
        names[(L.FFN_W2, i)] = f"{p}.feed_forward.w2.weight"
        names[(L.FFN_W3, i)] = f"{p}.feed_forward.w3.weight"
        names[(L.FFN_NORM, i)] = f"{p}.ffn_norm.weight"
        names[(L.OPERATOR_NORM, i)] = f"{p}.operator_norm.weight"
    return names


LEVELS = {"ternary": "ternary-v1", "nf4": "nf4-v1", "int8": "int8-v1"}


def write_lfm2_bundle(path, cfg, host: dict) -> None:
    """Write `host` ({(role, layer): arrays} as synthetic_host_weights
    yields them) as a `minifield.mixed.v1` safetensors bundle."""
    from safetensors.numpy import save_file

    from . import convert
    from . import lfm2 as L
    tensors, levels = {}, {}
    for key, name in lfm2_tensor_names(cfg).items():
        arrays = host[key]
        if len(arrays) == 2:
            codes, scales = arrays
            tensors[name + ".codes"] = np.ascontiguousarray(codes, dtype=np.uint8)
            half = np.asarray(scales, dtype=np.float32).astype(np.float16)
            assert np.array_equal(convert.f16_to_f32(half), scales), "scales must be binary16"
            tensors[name + ".scales"] = half
            fmt = {4: "ternary", 2: "nf4", 1: "int8"}[scales.shape[1] * 128 // codes.shape[1]]
            levels[name] = LEVELS[fmt]
        else:
            (values,) = arrays
            if key[0] == L.CONV_KERNEL:
                values = values.reshape(values.shape[0], 1, values.shape[1])
            tensors[name] = np.ascontiguousarray(values, dtype=np.float32)
            if key[0] in (L.TOKEN_EMBEDDING, L.CONV_IN, L.CONV_OUT, L.QUERY, L.KEY, L.VALUE,
                          L.OUTPUT, L.FFN_W1, L.FFN_W2, L.FFN_W3):
                levels[name] = "f32"
    metadata = {"format": "minifield.mixed.v1", "tensor_quantization": json.dumps(levels),
                "group_size": "128"}
    save_file(tensors, str(path), metadata=metadata)


__all__ = ["SafetensorsFile", "load_lfm2", "lfm2_tensor_names", "write_lfm2_bundle"]
