"""ctypes declarations of the C ABI in include/minifield_hip.h and
include/minifield_convert.h.

The library is the in-tree build `runtime_amd/libminifield_hip.so`.  Loading
fails loudly when it is missing: there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import pathlib

LIBRARY_PATH = pathlib.Path(__file__).resolve().parent / "libminifield_hip.so"

c_u64_p = ctypes.POINTER(ctypes.c_uint64)
c_u32_p = ctypes.POINTER(ctypes.c_uint32)
c_float_p = ctypes.POINTER(ctypes.c_float)
c_u8_p = ctypes.POINTER(ctypes.c_uint8)
c_u16_p = ctypes.POINTER(ctypes.c_uint16)


class Limits(ctypes.Structure):
    _fields_ = [("max_allocation_bytes", ctypes.c_uint64),
                ("max_total_bytes", ctypes.c_uint64),
                ("max_pending_operations", ctypes.c_uint32)]


class BackendIdentity(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_uint32), ("ordinal", ctypes.c_uint32),
                ("owner", ctypes.c_uint64), ("generation", ctypes.c_uint64)]


class BackendCapabilities(ctypes.Structure):
    _fields_ = [("dtypes", ctypes.c_uint32), ("operations", ctypes.c_uint64),
                ("max_rank", ctypes.c_uint32), ("max_elements", ctypes.c_uint64),
                ("max_allocation_bytes", ctypes.c_uint64),
                ("supports_nonblocking_completion", ctypes.c_uint32)]


class Report(ctypes.Structure):
    _fields_ = [("resident_weight_bytes", ctypes.c_uint64), ("cache_bytes", ctypes.c_uint64),
                ("scratch_bytes", ctypes.c_uint64), ("staged_branch_bytes", ctypes.c_uint64),
                ("pending_operation_bytes", ctypes.c_uint64),
                ("pending_operations", ctypes.c_uint32)]


class MflConfig(ctypes.Structure):
    """mfl_config (include/minifield_lfm2.h)."""
    _fields_ = [("hidden", ctypes.c_uint32), ("intermediate", ctypes.c_uint32),
                ("attention_heads", ctypes.c_uint32), ("key_value_heads", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("conv_width", ctypes.c_uint32),
                ("vocab", ctypes.c_uint32), ("layer_count", ctypes.c_uint32),
                ("layer_kinds", ctypes.POINTER(ctypes.c_uint8)), ("rope_theta", ctypes.c_float),
                ("norm_epsilon", ctypes.c_float), ("block_norm_epsilon", ctypes.c_float),
                ("max_tokens", ctypes.c_uint64)]


P = ctypes.c_void_p
PP = ctypes.POINTER(ctypes.c_void_p)
S = ctypes.c_int  # mfh_status
SZ = ctypes.c_size_t

# name -> (restype, argtypes).  Kept in the header's order; tests check that
# every symbol declared in include/*.h is exported and described here.
SIGNATURES = {
    # context
    "mfh_create": (S, [ctypes.c_uint32, ctypes.c_uint64, ctypes.POINTER(Limits), PP]),
    "mfh_destroy": (None, [P]),
    "mfh_last_error": (ctypes.c_char_p, [P]),
    "mfh_status_message": (ctypes.c_char_p, [S]),
    "mfh_identity": (S, [P, ctypes.POINTER(BackendIdentity)]),
    "mfh_capabilities": (S, [P, ctypes.POINTER(BackendCapabilities)]),
    "mfh_resource_report": (S, [P, ctypes.POINTER(Report)]),
    "mfh_peak_accounted_bytes": (S, [P, c_u64_p]),
    "mfh_advance_generation": (S, [P]),
    "mfh_request_cancel": (S, [P]),
    "mfh_clear_cancel": (S, [P]),
    "mfh_poll_retired_fences": (S, [P]),
    # buffers
    "mfh_alloc_f32": (S, [P, c_u64_p, ctypes.c_uint32, ctypes.c_int, ctypes.c_int, PP]),
    "mfh_upload_f32": (S, [P, c_u64_p, ctypes.c_uint32, c_float_p, SZ, ctypes.c_int, PP]),
    "mfh_upload_u8": (S, [P, c_u64_p, ctypes.c_uint32, c_u8_p, SZ, ctypes.c_int, PP]),
    "mfh_release": (None, [P]),
    "mfh_buf_desc": (S, [P, ctypes.POINTER(ctypes.c_int), c_u32_p, c_u64_p]),
    # completions
    "mfh_fence_submit": (S, [P, PP]),
    "mfh_fence_poll": (S, [P, ctypes.POINTER(ctypes.c_int)]),
    "mfh_fence_cancel": (S, [P]),
    "mfh_fence_free": (None, [P]),
    "mfh_read_f32_async": (S, [P, P, PP]),
    "mfh_readback_poll": (S, [P, ctypes.POINTER(ctypes.c_int), c_float_p, SZ,
                              ctypes.POINTER(SZ)]),
    "mfh_readback_cancel": (S, [P]),
    "mfh_readback_free": (None, [P]),
    "mfh_synchronize": (S, [P]),
    # packed ops
    "mfh_packed_gather_rows": (S, [P, P, P, P, c_u32_p, SZ, P]),
    "mfh_packed_linear": (S, [P, P, P, P, P]),
    "mfh_packed_linear_pair": (S, [P, P, P, P, P, P, P, P]),
    "mfh_packed_swiglu_linear": (S, [P, P, P, P, P, P]),
    "mfh_packed_swiglu_pair": (S, [P, P, P, P, P, P, P]),
    "mfh_prepare_packed": (S, [P, P, P]),
    "mfh_packed_prepared": (ctypes.c_int, [P, P, P]),
    "mfh_supports_ternary_lut2": (ctypes.c_int, [P]),
    "mfh_packed_linear_noalloc": (S, [P, P, P, P, P]),
    # dense ops
    "mfh_copy": (S, [P, P, P]),
    "mfh_copy_rect_2d": (S, [P, P, P] + [ctypes.c_uint64] * 6),
    "mfh_argmax": (S, [P, P, P]),
    "mfh_argmax_masked": (S, [P, P, P, c_u64_p, SZ]),
    "mfh_gather_rows": (S, [P, P, P, c_u32_p, SZ, P]),
    "mfh_gather_columns": (S, [P, P, P, c_u32_p, SZ]),
    "mfh_add": (S, [P, P, P, P]),
    "mfh_multiply": (S, [P, P, P, P]),
    "mfh_linear": (S, [P, P, P, P]),
    "mfh_row_rms_norm": (S, [P, P, P, P, ctypes.c_float]),
    "mfh_head_rms_norm": (S, [P, P, P, P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float]),
    "mfh_split_half_rotary": (S, [P, P, P, c_u64_p, SZ, ctypes.c_uint32, ctypes.c_uint32,
                                  ctypes.c_float]),
    "mfh_add_row_rms_norm": (S, [P, P, P, P, P, P, ctypes.c_float]),
    "mfh_qk_norm_rope": (S, [P, P, P, P, P, P, P, c_u64_p, SZ, ctypes.c_uint32, ctypes.c_uint32,
                             ctypes.c_float, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float]),
    "mfh_causal_gqa": (S, [P, P, P, P, P, P, P, c_u64_p, ctypes.c_uint32, ctypes.c_uint32,
                           ctypes.c_uint32]),
    "mfh_gated_short_convolution": (S, [P, P, P, P, P, ctypes.c_uint32, ctypes.c_uint32]),
    "mfh_swiglu": (S, [P, P, P, P]),
    # LFM2 token pass (minifield_lfm2.h)
    "mfl_create": (S, [P, ctypes.POINTER(MflConfig), PP]),
    "mfl_destroy": (None, [P]),
    "mfl_set_weight": (S, [P, ctypes.c_uint32, ctypes.c_uint32, P, P]),
    "mfl_reset": (S, [P]),
    "mfl_length": (ctypes.c_uint64, [P]),
    "mfl_append": (S, [P, c_u32_p, SZ, P, ctypes.c_int]),
    "mfl_sample": (S, [P]),
    "mfl_generate": (S, [P, ctypes.c_uint32, P]),
    "mfl_logits": (P, [P]),
    "mfl_sampled": (P, [P]),
    "mfl_snapshot": (S, [P, PP]),
    "mfl_restore": (S, [P, P]),
    "mfl_prefix_length": (ctypes.c_uint64, [P]),
    "mfl_prefix_destroy": (None, [P]),
    # safetensors loader (minifield_loader.h)
    "mfs_open": (S, [ctypes.c_char_p, ctypes.c_uint64, PP]),
    "mfs_close": (None, [P]),
    "mfs_error": (ctypes.c_char_p, []),
    "mfs_tensor_count": (SZ, [P]),
    "mfs_tensor_name": (ctypes.c_char_p, [P, SZ]),
    "mfs_tensor_info": (S, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int), c_u32_p, c_u64_p]),
    "mfs_metadata": (ctypes.c_char_p, [P, ctypes.c_char_p]),
    "mfs_matmul_scheme": (S, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)]),
    "mfs_upload_packed": (S, [P, P, ctypes.c_char_p, ctypes.c_int, PP, PP]),
    "mfs_upload_dense": (S, [P, P, ctypes.c_char_p, ctypes.c_int, PP]),
    "mfl_load_safetensors": (S, [P, P]),
    # diagnostics
    "mfh_stream": (P, [P]),
    "mfh_set_kernel_path": (ctypes.c_int, [P, ctypes.c_int]),
    "mfh_set_gemm_activations": (ctypes.c_int, [P, ctypes.c_int]),
    # converters
    "mfc_quantize": (ctypes.c_int, [c_float_p, SZ, SZ, ctypes.c_int, c_u8_p, c_u16_p,
                                    ctypes.c_uint]),
    "mfc_dequantize": (ctypes.c_int, [c_u8_p, c_u16_p, SZ, SZ, ctypes.c_int, c_float_p]),
    "mfc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "mfc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
    "mfc_f16_to_f32_array": (None, [c_u16_p, c_float_p, SZ]),
    "mfc_fill_normal": (None, [c_float_p, SZ, ctypes.c_uint64, ctypes.c_double, ctypes.c_double,
                               ctypes.c_uint]),
    "mfc_fill_token_ids": (None, [c_u32_p, SZ, ctypes.c_uint64, ctypes.c_uint32]),
}

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Load the built library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIBRARY_PATH.exists():
            raise RuntimeError(
                f"{LIBRARY_PATH} is missing: build it with `python -m runtime_amd.build`"
            )
        handle = ctypes.CDLL(str(LIBRARY_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib
