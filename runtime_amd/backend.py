"""`HipBackend`: the Python host mirror of the reference's `InferenceOps`
contract (crates/engine-api/src/inference.rs:33-425) over the C ABI.

Method names, operand order and error behaviour follow the trait: every
method raises `ExecutorError` carrying the C status's variant name and the
static message the library reported, and a rejected call leaves its outputs
untouched.  Buffers are opaque handles owned by one backend instance and
generation.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Sequence

import numpy as np

from . import _ffi

# ExecutorError variants in declaration order (engine-api/src/error.rs:10-28).
VARIANTS = [
    "Ok", "InvalidArgument", "InvalidShape", "InvalidLayout", "InvalidDType", "Overflow",
    "OutOfBounds", "Unsupported", "ResourceLimit", "WrongBackend", "StaleBuffer",
    "DuplicateName", "MissingRequiredTensor", "UnexpectedTensor", "InvalidTie", "Cancelled",
    "CompletionConsumed", "BackendFailure",
]

# AllocationClass (engine-api/src/resources.rs:19-24).
WEIGHT, CACHE, SCRATCH, BRANCH = 0, 1, 2, 3
F32, U8 = 0, 1


class ExecutorError(Exception):
    """A failed backend call: `variant` names the ExecutorError variant."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.variant = VARIANTS[status] if 0 <= status < len(VARIANTS) else f"Status{status}"
        self.message = message
        super().__init__(f"{self.variant}: {message}")


@dataclass(frozen=True)
class Limits:
    max_allocation_bytes: int = 1 << 40
    max_total_bytes: int = 1 << 41
    max_pending_operations: int = 1 << 20


class Buffer:
    """Opaque device buffer handle; released when garbage collected."""

    __slots__ = ("_handle", "_backend", "dtype", "shape")

    def __init__(self, handle: int, backend: "HipBackend", dtype: int, shape: tuple[int, ...]):
        self._handle = handle
        self._backend = backend
        self.dtype = dtype
        self.shape = shape

    @property
    def handle(self) -> int:
        return self._handle

    def release(self) -> None:
        if self._handle:
            _ffi.lib().mfh_release(self._handle)
            self._handle = 0

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


def _dims(shape: Sequence[int]):
    arr = (ctypes.c_uint64 * max(1, len(shape)))(*[int(d) for d in shape])
    return arr, len(shape)


def _h(buf: Buffer | None) -> int | None:
    return None if buf is None else buf.handle


class Fence:
    def __init__(self, handle: int, backend: "HipBackend"):
        self._handle = handle
        self._backend = backend

    def poll_step(self) -> bool:
        """Return True once ready; raise ExecutorError if the fence failed."""
        ready = ctypes.c_int(0)
        status = _ffi.lib().mfh_fence_poll(self._handle, ctypes.byref(ready))
        if status:
            raise ExecutorError(status, self._backend.last_error())
        return bool(ready.value)

    def cancel(self) -> None:
        _ffi.lib().mfh_fence_cancel(self._handle)

    def __del__(self):
        try:
            if self._handle:
                _ffi.lib().mfh_fence_free(self._handle)
                self._handle = 0
        except Exception:
            pass


class Readback:
    def __init__(self, handle: int, backend: "HipBackend", count: int):
        self._handle = handle
        self._backend = backend
        self._count = count

    def poll_step(self) -> np.ndarray | None:
        """Return the values once ready (None while pending)."""
        ready = ctypes.c_int(0)
        out = np.empty(self._count, dtype=np.float32)
        got = ctypes.c_size_t(0)
        status = _ffi.lib().mfh_readback_poll(
            self._handle, ctypes.byref(ready),
            out.ctypes.data_as(_ffi.c_float_p), out.size, ctypes.byref(got))
        if status:
            raise ExecutorError(status, self._backend.last_error())
        return out if ready.value else None

    def cancel(self) -> None:
        _ffi.lib().mfh_readback_cancel(self._handle)

    def __del__(self):
        try:
            if self._handle:
                _ffi.lib().mfh_readback_free(self._handle)
                self._handle = 0
        except Exception:
            pass


class HipBackend:
    """One backend instance on one HIP device (one stream)."""

    def __init__(self, ordinal: int = 0, owner: int = 1, limits: Limits = Limits()):
        lib = _ffi.lib()
        handle = ctypes.c_void_p()
        c_limits = _ffi.Limits(limits.max_allocation_bytes, limits.max_total_bytes,
                               limits.max_pending_operations)
        status = lib.mfh_create(ordinal, owner, ctypes.byref(c_limits), ctypes.byref(handle))
        if status:
            raise ExecutorError(status, lib.mfh_status_message(status).decode())
        self._ctx = handle.value

    # -- lifetime ---------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_ctx", None):
            _ffi.lib().mfh_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def ctx(self) -> int:
        return self._ctx

    def last_error(self) -> str:
        return _ffi.lib().mfh_last_error(self._ctx).decode()

    def _check(self, status: int) -> None:
        if status:
            raise ExecutorError(status, self.last_error())

    # -- identity, capabilities, accounting ----------------------------------
    def identity(self) -> _ffi.BackendIdentity:
        out = _ffi.BackendIdentity()
        self._check(_ffi.lib().mfh_identity(self._ctx, ctypes.byref(out)))
        return out

    def capabilities(self) -> _ffi.BackendCapabilities:
        out = _ffi.BackendCapabilities()
        self._check(_ffi.lib().mfh_capabilities(self._ctx, ctypes.byref(out)))
        return out

    def resource_report(self) -> _ffi.Report:
        out = _ffi.Report()
        self._check(_ffi.lib().mfh_resource_report(self._ctx, ctypes.byref(out)))
        return out

    def peak_accounted_bytes(self) -> int:
        out = ctypes.c_uint64(0)
        self._check(_ffi.lib().mfh_peak_accounted_bytes(self._ctx, ctypes.byref(out)))
        return out.value

    def advance_generation(self) -> None:
        self._check(_ffi.lib().mfh_advance_generation(self._ctx))

    def request_cancel(self) -> None:
        self._check(_ffi.lib().mfh_request_cancel(self._ctx))

    def clear_cancel(self) -> None:
        self._check(_ffi.lib().mfh_clear_cancel(self._ctx))

    def poll_retired_fences(self) -> None:
        self._check(_ffi.lib().mfh_poll_retired_fences(self._ctx))

    def supports_ternary_lut2(self) -> bool:
        return bool(_ffi.lib().mfh_supports_ternary_lut2(self._ctx))

    def set_kernel_path(self, path: int) -> int:
        """0 automatic, 1 FP32 FMA kernels only, 2 matrix-core kernels only."""
        return _ffi.lib().mfh_set_kernel_path(self._ctx, path)

    def set_gemm_activations(self, mode: int) -> int:
        """Prefill GEMM activations: 0 binary16 hi + lo (default), 1 one half."""
        return _ffi.lib().mfh_set_gemm_activations(self._ctx, mode)

    def stream(self) -> int:
        return _ffi.lib().mfh_stream(self._ctx)

    # -- buffers ------------------------------------------------------------
    def allocate_f32_classified(self, shape: Sequence[int], cls: int = SCRATCH) -> Buffer:
        return self._alloc(shape, cls, zeroed=1)

    def allocate_f32(self, shape: Sequence[int]) -> Buffer:
        return self._alloc(shape, SCRATCH, zeroed=1)

    def allocate_f32_uninit(self, shape: Sequence[int], cls: int = SCRATCH) -> Buffer:
        return self._alloc(shape, cls, zeroed=0)

    def _alloc(self, shape, cls, zeroed) -> Buffer:
        dims, rank = _dims(shape)
        out = ctypes.c_void_p()
        self._check(_ffi.lib().mfh_alloc_f32(self._ctx, dims, rank, cls, zeroed,
                                             ctypes.byref(out)))
        return Buffer(out.value, self, F32, tuple(int(d) for d in shape))

    def upload_f32_classified(self, shape: Sequence[int], values, cls: int = SCRATCH) -> Buffer:
        arr = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
        dims, rank = _dims(shape)
        out = ctypes.c_void_p()
        self._check(_ffi.lib().mfh_upload_f32(self._ctx, dims, rank,
                                              arr.ctypes.data_as(_ffi.c_float_p), arr.size, cls,
                                              ctypes.byref(out)))
        return Buffer(out.value, self, F32, tuple(int(d) for d in shape))

    def upload_f32(self, shape: Sequence[int], values) -> Buffer:
        return self.upload_f32_classified(shape, values, SCRATCH)

    def upload_u8_classified(self, shape: Sequence[int], values, cls: int = WEIGHT) -> Buffer:
        arr = np.ascontiguousarray(values, dtype=np.uint8).reshape(-1)
        dims, rank = _dims(shape)
        out = ctypes.c_void_p()
        self._check(_ffi.lib().mfh_upload_u8(self._ctx, dims, rank,
                                             arr.ctypes.data_as(_ffi.c_u8_p), arr.size, cls,
                                             ctypes.byref(out)))
        return Buffer(out.value, self, U8, tuple(int(d) for d in shape))

    # -- completions ----------------------------------------------------------
    def fence(self) -> Fence:
        out = ctypes.c_void_p()
        self._check(_ffi.lib().mfh_fence_submit(self._ctx, ctypes.byref(out)))
        return Fence(out.value, self)

    def read_f32_async(self, buf: Buffer) -> Readback:
        out = ctypes.c_void_p()
        self._check(_ffi.lib().mfh_read_f32_async(self._ctx, buf.handle, ctypes.byref(out)))
        count = int(np.prod(buf.shape)) if buf.shape else 1
        return Readback(out.value, self, count)

    def read(self, buf: Buffer) -> np.ndarray:
        """Submit a readback and poll it to completion (test convenience)."""
        rb = self.read_f32_async(buf)
        while True:
            values = rb.poll_step()
            if values is not None:
                return values.reshape(buf.shape)

    def synchronize(self) -> None:
        self._check(_ffi.lib().mfh_synchronize(self._ctx))

    # -- packed operations (inference.rs:180-252) ---------------------------
    def packed_gather_rows(self, output: Buffer, codes: Buffer, scales: Buffer, ids) -> None:
        """`ids` is a host sequence of u32 ids (TokenIds::Host) or a device
        f32 rank-1 Buffer (TokenIds::Device)."""
        lib = _ffi.lib()
        if isinstance(ids, Buffer):
            self._check(lib.mfh_packed_gather_rows(self._ctx, output.handle, codes.handle,
                                                   scales.handle, None, 0, ids.handle))
        else:
            host = np.ascontiguousarray(ids, dtype=np.uint32).reshape(-1)
            ptr = host.ctypes.data_as(_ffi.c_u32_p) if host.size else None
            self._check(lib.mfh_packed_gather_rows(self._ctx, output.handle, codes.handle,
                                                   scales.handle, ptr, host.size, None))

    def prepare_packed(self, codes: Buffer, scales: Buffer) -> None:
        """Build the pair's private tile copies now (mfh_prepare_packed)."""
        self._check(_ffi.lib().mfh_prepare_packed(self._ctx, codes.handle, scales.handle))

    def packed_prepared(self, codes: Buffer, scales: Buffer) -> bool:
        return bool(_ffi.lib().mfh_packed_prepared(self._ctx, codes.handle, scales.handle))

    def packed_linear(self, output: Buffer, input: Buffer, codes: Buffer, scales: Buffer) -> None:
        self._check(_ffi.lib().mfh_packed_linear(self._ctx, output.handle, input.handle,
                                                 codes.handle, scales.handle))

    def packed_linear_noalloc(self, output: Buffer, input: Buffer, codes: Buffer,
                              scales: Buffer) -> None:
        """packed_linear without device allocation (mfh_packed_linear_noalloc)."""
        self._check(_ffi.lib().mfh_packed_linear_noalloc(self._ctx, output.handle, input.handle,
                                                         codes.handle, scales.handle))

    def packed_linear_pair(self, out_a: Buffer, out_b: Buffer, input: Buffer, codes_a: Buffer,
                           scales_a: Buffer, codes_b: Buffer, scales_b: Buffer) -> None:
        self._check(_ffi.lib().mfh_packed_linear_pair(
            self._ctx, out_a.handle, out_b.handle, input.handle, codes_a.handle,
            scales_a.handle, codes_b.handle, scales_b.handle))

    def packed_swiglu_linear(self, output: Buffer, gate: Buffer, up: Buffer, codes: Buffer,
                             scales: Buffer) -> None:
        self._check(_ffi.lib().mfh_packed_swiglu_linear(
            self._ctx, output.handle, gate.handle, up.handle, codes.handle, scales.handle))

    def packed_swiglu_pair(self, output: Buffer, input: Buffer, codes_a: Buffer,
                           scales_a: Buffer, codes_b: Buffer, scales_b: Buffer) -> None:
        self._check(_ffi.lib().mfh_packed_swiglu_pair(
            self._ctx, output.handle, input.handle, codes_a.handle, scales_a.handle,
            codes_b.handle, scales_b.handle))

    # ---- dense ops (inference.rs:113-424) --------------------------------

    def copy(self, output: Buffer, input: Buffer) -> None:
        self._check(_ffi.lib().mfh_copy(self._ctx, output.handle, input.handle))

    def copy_rect_2d(self, output: Buffer, input: Buffer, rect: "RectCopy2d") -> None:
        self._check(_ffi.lib().mfh_copy_rect_2d(
            self._ctx, output.handle, input.handle, rect.source_row, rect.source_column,
            rect.destination_row, rect.destination_column, rect.rows, rect.columns))

    def argmax(self, output: Buffer, input: Buffer) -> None:
        self._check(_ffi.lib().mfh_argmax(self._ctx, output.handle, input.handle))

    def argmax_masked(self, output: Buffer, input: Buffer, mask) -> None:
        words = np.ascontiguousarray(mask, dtype=np.uint64).reshape(-1)
        ptr = words.ctypes.data_as(_ffi.c_u64_p) if words.size else None
        self._check(_ffi.lib().mfh_argmax_masked(self._ctx, output.handle, input.handle, ptr,
                                                 words.size))

    def gather_rows(self, output: Buffer, table: Buffer, ids) -> None:
        """`ids` as for `packed_gather_rows`."""
        lib = _ffi.lib()
        if isinstance(ids, Buffer):
            self._check(lib.mfh_gather_rows(self._ctx, output.handle, table.handle, None, 0,
                                            ids.handle))
        else:
            host = np.ascontiguousarray(ids, dtype=np.uint32).reshape(-1)
            ptr = host.ctypes.data_as(_ffi.c_u32_p) if host.size else None
            self._check(lib.mfh_gather_rows(self._ctx, output.handle, table.handle, ptr,
                                            host.size, None))

    def gather_columns(self, output: Buffer, input: Buffer, columns) -> None:
        cols = np.ascontiguousarray(columns, dtype=np.uint32).reshape(-1)
        ptr = cols.ctypes.data_as(_ffi.c_u32_p) if cols.size else None
        self._check(_ffi.lib().mfh_gather_columns(self._ctx, output.handle, input.handle, ptr,
                                                  cols.size))

    def add(self, output: Buffer, left: Buffer, right: Buffer) -> None:
        self._check(_ffi.lib().mfh_add(self._ctx, output.handle, left.handle, right.handle))

    def multiply(self, output: Buffer, left: Buffer, right: Buffer) -> None:
        self._check(_ffi.lib().mfh_multiply(self._ctx, output.handle, left.handle,
                                            right.handle))

    def linear(self, output: Buffer, input: Buffer, weight: Buffer) -> None:
        self._check(_ffi.lib().mfh_linear(self._ctx, output.handle, input.handle,
                                          weight.handle))

    def row_rms_norm(self, output: Buffer, input: Buffer, weight: Buffer, epsilon: float) -> None:
        self._check(_ffi.lib().mfh_row_rms_norm(self._ctx, output.handle, input.handle,
                                                weight.handle, epsilon))

    def head_rms_norm(self, output: Buffer, input: Buffer, weight: Buffer,
                      heads: "PackedHeadSpec", epsilon: float) -> None:
        self._check(_ffi.lib().mfh_head_rms_norm(self._ctx, output.handle, input.handle,
                                                 weight.handle, heads.heads, heads.head_dim,
                                                 epsilon))

    def split_half_rotary(self, output: Buffer, input: Buffer, positions,
                          spec: "RotarySpec") -> None:
        pos = np.ascontiguousarray(positions, dtype=np.uint64).reshape(-1)
        ptr = pos.ctypes.data_as(_ffi.c_u64_p) if pos.size else None
        self._check(_ffi.lib().mfh_split_half_rotary(
            self._ctx, output.handle, input.handle, ptr, pos.size, spec.heads.heads,
            spec.heads.head_dim, spec.theta))

    def add_row_rms_norm(self, sum: Buffer, normed: Buffer, left: Buffer, right: Buffer,
                         weight: Buffer, epsilon: float) -> None:
        self._check(_ffi.lib().mfh_add_row_rms_norm(self._ctx, sum.handle, normed.handle,
                                                    left.handle, right.handle, weight.handle,
                                                    epsilon))

    def qk_norm_rope(self, query_out: Buffer, key_out: Buffer, query: Buffer, key: Buffer,
                     query_weight: Buffer, key_weight: Buffer, positions, rope: "RotarySpec",
                     key_value_heads: "PackedHeadSpec", epsilon: float) -> None:
        pos = np.ascontiguousarray(positions, dtype=np.uint64).reshape(-1)
        ptr = pos.ctypes.data_as(_ffi.c_u64_p) if pos.size else None
        self._check(_ffi.lib().mfh_qk_norm_rope(
            self._ctx, query_out.handle, key_out.handle, query.handle, key.handle,
            query_weight.handle, key_weight.handle, ptr, pos.size, rope.heads.heads,
            rope.heads.head_dim, rope.theta, key_value_heads.heads, key_value_heads.head_dim,
            epsilon))

    def causal_gqa(self, output: Buffer, query: Buffer, key: Buffer, value: Buffer,
                   key_cache: Buffer, value_cache: Buffer, cache_len: "CacheLength",
                   spec: "GqaSpec") -> None:
        """`cache_len` is a mutable `CacheLength`; it advances only on success."""
        length = ctypes.c_uint64(cache_len.value)
        self._check(_ffi.lib().mfh_causal_gqa(
            self._ctx, output.handle, query.handle, key.handle, value.handle, key_cache.handle,
            value_cache.handle, ctypes.byref(length), spec.query_heads, spec.key_value_heads,
            spec.head_dim))
        cache_len.value = length.value

    def gated_short_convolution(self, output: Buffer, projection: Buffer, kernel: Buffer,
                                history: Buffer, spec: "GatedShortConvSpec") -> None:
        self._check(_ffi.lib().mfh_gated_short_convolution(
            self._ctx, output.handle, projection.handle, kernel.handle, history.handle,
            spec.hidden, spec.width))

    def swiglu(self, output: Buffer, gate: Buffer, up: Buffer) -> None:
        self._check(_ffi.lib().mfh_swiglu(self._ctx, output.handle, gate.handle, up.handle))


# ---- operation descriptors (engine-api/src/backend.rs:128-383) -------------
# Plain carriers: the library validates them with the reference's rules and
# messages when an operation receives them.

@dataclass(frozen=True)
class RectCopy2d:
    source_row: int
    source_column: int
    destination_row: int
    destination_column: int
    rows: int
    columns: int


@dataclass(frozen=True)
class PackedHeadSpec:
    heads: int
    head_dim: int


@dataclass(frozen=True)
class RotarySpec:
    heads: PackedHeadSpec
    theta: float


@dataclass(frozen=True)
class GqaSpec:
    query_heads: int
    key_value_heads: int
    head_dim: int


@dataclass(frozen=True)
class GatedShortConvSpec:
    hidden: int
    width: int


@dataclass
class CacheLength:
    """The `&mut u64` cache length of `causal_gqa`."""
    value: int = 0
