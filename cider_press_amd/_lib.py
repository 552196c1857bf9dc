"""ctypes binding of libcpq.so (the HIP library; C ABI in include/cpq.h).

There is no fallback: if the shared library is missing this module raises,
so nothing silently runs on the CPU.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcpq.so")

# cpq_status
OK = 0
NO_DEVICE = 1
KERNEL_NOT_FOUND = 2
BUFFER_ALLOCATION = 3
BUFFER_TOO_LARGE = 4
INVALID_ARGUMENT = 5
COMMAND_BUFFER_FAILED = 6
HIP_API = 7
MISSING_KEY = 8
UNSUPPORTED_DTYPE = 9
SHAPE_MISMATCH = 10
SAFETENSORS = 11
JSON = 12

# cpq_dtype
DTYPES = {"f32": 0, "f16": 1, "bf16": 2, "u32": 3}


class Error(Exception):
    """cider_press_kernels::Error analogue; `kind` names the variant."""

    kind = "Error"

    def __init__(self, message: str):
        super().__init__(message)
        self.message = message


class NoDevice(Error):
    kind = "NoDevice"


class KernelNotFound(Error):
    kind = "KernelNotFound"


class BufferAllocation(Error):
    kind = "BufferAllocation"


class BufferTooLarge(Error):
    kind = "BufferTooLarge"


class InvalidArgument(Error):
    kind = "InvalidArgument"


class CommandBufferFailed(Error):
    kind = "CommandBufferFailed"


class HipApi(Error):
    kind = "HipApi"


# Loader errors (cider-press-models/src/error.rs:9-60).
class MissingKey(Error):
    kind = "MissingKey"


class UnsupportedDtype(Error):
    kind = "UnsupportedDtype"


class ShapeMismatch(Error):
    kind = "ShapeMismatch"


class SafetensorsError(Error):
    kind = "Safetensors"


class JsonError(Error):
    kind = "Json"


_ERRORS = {
    NO_DEVICE: NoDevice,
    KERNEL_NOT_FOUND: KernelNotFound,
    BUFFER_ALLOCATION: BufferAllocation,
    BUFFER_TOO_LARGE: BufferTooLarge,
    INVALID_ARGUMENT: InvalidArgument,
    COMMAND_BUFFER_FAILED: CommandBufferFailed,
    HIP_API: HipApi,
    MISSING_KEY: MissingKey,
    UNSUPPORTED_DTYPE: UnsupportedDtype,
    SHAPE_MISMATCH: ShapeMismatch,
    SAFETENSORS: SafetensorsError,
    JSON: JsonError,
}

_c = ctypes
_vp = _c.c_void_p
_sz = _c.c_size_t
_u32 = _c.c_uint32
_int = _c.c_int
_st = _c.c_int  # cpq_status
_pp = _c.POINTER(_c.c_void_p)
_psz = _c.POINTER(_c.c_size_t)

# name -> (restype, argtypes); the full ABI of include/cpq.h
SIGNATURES = {
    "cpq_last_error_message": (_c.c_char_p, []),
    "cpq_version": (_c.c_char_p, []),
    "cpq_device_system_default": (_st, [_pp]),
    "cpq_device_release": (None, [_vp]),
    "cpq_device_info": (_st, [_vp, _c.c_char_p, _sz, _c.POINTER(_int), _c.POINTER(_int)]),
    "cpq_alloc_buffer": (_st, [_vp, _sz, _pp, _psz]),
    "cpq_upload": (_st, [_vp, _vp, _sz, _pp, _psz]),
    "cpq_free_buffer": (_st, [_vp, _vp]),
    "cpq_read_buffer": (_st, [_vp, _vp, _vp, _sz]),
    "cpq_write_buffer": (_st, [_vp, _vp, _vp, _sz]),
    "cpq_commands_create": (_st, [_vp, _pp]),
    "cpq_commands_wrap_stream": (_st, [_vp, _vp, _pp]),
    "cpq_commands_stream": (_vp, [_vp]),
    "cpq_commands_commit": (_st, [_vp]),
    "cpq_commands_wait": (_st, [_vp]),
    "cpq_commands_commit_and_wait": (_st, [_vp]),
    "cpq_commands_release": (None, [_vp]),
    "cpq_commands_begin_capture": (_st, [_vp]),
    "cpq_commands_end_capture": (_st, [_vp, _pp]),
    "cpq_graph_launch": (_st, [_vp, _vp]),
    "cpq_graph_release": (None, [_vp]),
    "cpq_commands_record_input": (_st, [_vp, _c.c_uint64]),
    "cpq_commands_record_output": (_st, [_vp, _c.c_uint64]),
    "cpq_commands_record_unresolved_input": (_st, [_vp]),
    "cpq_commands_elide_next_barrier": (_st, [_vp]),
    "cpq_device_supports_stage_boundary_sampling": (_int, [_vp]),
    "cpq_device_gpu_timestamp_period_ns": (_st, [_vp, _c.POINTER(_c.c_double)]),
    "cpq_commands_create_profiled": (_st, [_vp, _sz, _pp]),
    "cpq_commands_begin_profiled_op": (_st, [_vp, _c.c_char_p]),
    "cpq_commands_profiled_info": (_st, [_vp, _psz, _psz]),
    "cpq_commands_commit_wait_resolve": (_st, [_vp, _vp, _sz, _psz]),
    "cpq_completion_result": (_st, [_int]),
    "cpq_event_create": (_st, [_pp]),
    "cpq_event_record": (_st, [_vp, _vp]),
    "cpq_event_elapsed_ms": (_st, [_vp, _vp, _c.POINTER(_c.c_float)]),
    "cpq_event_release": (None, [_vp]),
    "cpq_stream_read": (_st, [_vp, _c.POINTER(_vp), _c.POINTER(_sz), _int, _vp, _int]),
    "cpq_stream_read_variant": (_st, [_vp, _c.POINTER(_vp), _c.POINTER(_sz), _int, _vp, _int, _int]),
    "cpq_stream_read_variant_count": (_int, []),
    "cpq_quantization_validate": (_st, [_u32, _u32]),
    "cpq_packed_word_count": (_st, [_u32, _u32, _sz, _psz]),
    "cpq_group_count": (_st, [_u32, _u32, _sz, _psz]),
    "cpq_kernel_available": (_int, [_int, _u32, _u32]),
    "cpq_affine_qmv": (_st, [_vp, _int, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _u32, _u32]),
    "cpq_affine_qmm_t": (_st, [_vp, _int, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz,
                               _u32, _u32]),
    "cpq_affine_qmm_t_noalloc": (_st, [_vp, _int, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz,
                                       _u32, _u32]),
    "cpq_affine_dequantize": (_st, [_vp, _int, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _u32, _u32]),
    "cpq_affine_gather_qmm": (_st, [_vp, _int, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _vp, _sz, _vp, _sz,
                                    _sz, _sz, _sz, _u32, _u32, _int]),
    "cpq_quantized_matmul": (_st, [_vp, _int, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _vp, _sz, _sz, _sz,
                                   _u32, _u32]),
    "cpq_check_qmv_args": (_st, [_int, _sz, _sz, _sz, _sz, _sz, _sz, _u32, _u32]),
    "cpq_check_qmm_args": (_st, [_int, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _u32, _u32]),
    "cpq_check_dequantize_args": (_st, [_int, _sz, _sz, _sz, _sz, _u32, _u32]),
    "cpq_affine_qmm_t_batched": (_st, [_vp, _int, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz,
                                       _u32, _u32, _int, _c.POINTER(_int), _c.POINTER(_c.c_int64), _c.POINTER(_c.c_int64), _c.POINTER(_c.c_int64), _c.POINTER(_c.c_int64)]),
    "cpq_affine_qmv_batched": (_st, [_vp, _int, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz,
                                     _u32, _u32, _int, _c.POINTER(_int), _c.POINTER(_c.c_int64), _c.POINTER(_c.c_int64), _c.POINTER(_c.c_int64), _c.POINTER(_c.c_int64)]),
    "cpq_check_qmm_n_args": (_st, [_int, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _u32, _u32]),
    "cpq_affine_qmm_n": (_st, [_vp, _int, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz,
                               _u32, _u32]),
    "cpq_check_embed_args": (_st, [_int, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _u32, _u32]),
    "cpq_embed_tokens": (_st, [_vp, _int, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _vp, _sz, _u32, _u32]),
    "cpq_tensor_embed_tokens": (_st, [_vp, _vp, _pp]),
    "cpq_moe_route": (_st, [_vp, _int, _vp, _sz, _sz, _u32, _int, _vp, _vp, _vp, _vp, _vp, _vp]),
    "cpq_moe_combine": (_st, [_vp, _int, _vp, _sz, _vp, _vp, _sz, _u32, _sz, _vp, _sz]),
    "cpq_check_gather_args": (_st, [_int, _sz, _sz, _sz, _sz, _int, _sz, _sz, _sz, _sz, _sz, _u32, _u32]),
    "cpq_qweight_from_bytes": (_st, [_vp, _int, _sz, _sz, _sz, _u32, _u32, _vp, _sz, _vp, _sz, _vp, _sz, _pp]),
    "cpq_qweight_release": (None, [_vp]),
    "cpq_qweight_info": (_st, [_vp, _psz, _psz, _psz, _c.POINTER(_u32), _c.POINTER(_u32), _c.POINTER(_int)]),
    "cpq_safetensors_open": (_st, [_c.c_char_p, _pp]),
    "cpq_safetensors_deserialize": (_st, [_vp, _sz, _pp]),
    "cpq_safetensors_close": (None, [_vp]),
    "cpq_safetensors_len": (_st, [_vp, _psz]),
    "cpq_safetensors_name": (_st, [_vp, _sz, _c.POINTER(_c.c_char_p)]),
    "cpq_safetensors_tensor": (_st, [_vp, _c.c_char_p, _c.POINTER(_c.c_char_p), _psz, _sz, _psz, _pp, _psz]),
    "cpq_safetensors_metadata": (_st, [_vp, _c.c_char_p, _c.POINTER(_c.c_char_p)]),
    "cpq_read_quantized_weight": (_st, [_vp, _vp, _c.c_char_p, _u32, _u32, _pp]),
    "cpq_read_quantized_weight_k_padded": (_st, [_vp, _vp, _c.c_char_p, _u32, _u32, _sz, _pp]),
    "cpq_pad_quantized_k": (_st, [_vp, _vp, _vp, _sz, _sz, _sz, _u32, _u32, _sz, _vp, _vp, _vp]),
    "cpq_read_dense_tensor": (_st, [_vp, _vp, _c.c_char_p, _pp]),
    "cpq_quantization_from_config": (_st, [_c.c_char_p, _sz, _c.POINTER(_int), _c.POINTER(_u32),
                                           _c.POINTER(_u32)]),
    "cpq_tensor_from_host": (_st, [_vp, _int, _psz, _sz, _vp, _pp]),
    "cpq_tensor_quantized_matmul": (_st, [_vp, _vp, _int, _pp]),
    "cpq_tensor_dequantize": (_st, [_vp, _pp]),
    "cpq_tensor_eval": (_st, [_vp]),
    "cpq_tensor_shape": (_st, [_vp, _psz, _sz, _psz]),
    "cpq_tensor_read": (_st, [_vp, _vp, _sz]),
    "cpq_tensor_release": (None, [_vp]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load libcpq.so (built by ``python -m cider_press_amd._build``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m cider_press_amd._build` "
                "(the HIP library is required; there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    msg = lib().cpq_last_error_message()
    return msg.decode() if msg else ""


def check(status: int) -> None:
    if status != OK:
        raise _ERRORS.get(status, Error)(last_error())


def status_name(status: int) -> str:
    return {OK: "Ok"} .get(status) or _ERRORS.get(status, Error).kind
