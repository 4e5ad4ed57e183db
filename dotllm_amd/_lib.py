"""ctypes binding of libllmdot_hip.so (the C ABI in include/llmdot_hip.h).

The library is built in-tree (``dotllm_amd/libllmdot_hip.so``) by
``dotllm_amd.build.build()``.  There is no fallback: if the shared library is
missing or does not load, :func:`lib` raises.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libllmdot_hip.so")

# Status codes (include/llmdot_hip.h).
OK = 0
E_INVALID = -1
E_UNSUPPORTED = -2
E_NOT_FOUND = -3
E_RANGE = -4
E_DEVICE = -5
E_NOMEM = -6

# GgmlType (src/Llmdot.Core/Loading/GgmlType.cs:3-28).
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1 = 0, 1, 2, 3, 6, 7, 8, 9
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, BF16 = 10, 11, 12, 13, 14, 25
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q4_1: "Q4_1", Q5_0: "Q5_0", Q5_1: "Q5_1",
              Q8_0: "Q8_0", Q8_1: "Q8_1", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K",
              Q5_K: "Q5_K", Q6_K: "Q6_K", BF16: "BF16"}

# (elements per block, bytes per block): TensorSize.ByteCount (TensorSize.cs:7-24).
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22),
         Q5_1: (32, 24), Q8_0: (32, 34), Q8_1: (32, 40), Q2_K: (256, 84), Q3_K: (256, 110),
         Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}


def byte_count(ggml_type: int, elements: int) -> int:
    """TensorSize.ByteCount; raises NotImplementedError for unknown types (TensorSize.cs:23)."""
    if ggml_type not in BLOCK:
        raise NotImplementedError(f"Unsupported GGML type: {ggml_type}")
    be, bb = BLOCK[ggml_type]
    return elements // be * bb


class HipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class ModelDesc(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("layers", C.c_int32), ("heads", C.c_int32),
                ("kv_heads", C.c_int32), ("head_dim", C.c_int32), ("ffn", C.c_int32),
                ("vocab", C.c_int32), ("context", C.c_int32), ("rope_dim", C.c_int32),
                ("eps", C.c_float), ("rope_base", C.c_float), ("rope_linear_factor", C.c_float),
                ("kv_fp16", C.c_int32), ("bos", C.c_int32), ("sliding_window", C.c_int32),
                ("key_prefix", C.c_char_p)]


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("arch", C.c_char * 32), ("compute_units", C.c_int32),
                ("clock_mhz", C.c_int32), ("hbm_bytes", C.c_uint64)]


class Sampling(C.Structure):
    """llmdot_hip_sampling: SamplingOptions (SamplingOptions.cs:7-15) without the seed."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float),
                ("repeat_penalty", C.c_float), ("repeat_window", C.c_int32)]


class StepTiming(C.Structure):
    _fields_ = [("total_ms", C.c_float), ("gemv_ms", C.c_float), ("gemv_launches", C.c_int32),
                ("gemv_bytes", C.c_double)]


_P = C.c_void_p
_I32 = C.c_int32
_I64 = C.c_int64
_U32 = C.c_uint32
_U64 = C.c_uint64
_F = C.c_float
_S = C.c_char_p
_PI32 = C.POINTER(C.c_int32)
_PP = C.POINTER(C.c_void_p)

# name -> argtypes (all return int32 status unless noted)
SIGNATURES = {
    "llmdot_hip_device_count": [_PI32],
    "llmdot_hip_create": [_I32, _PP],
    "llmdot_hip_destroy": [_P],
    "llmdot_hip_get_device_info": [_P, C.POINTER(DeviceInfo)],
    "llmdot_hip_upload_weight": [_P, _S, _U32, _P, C.c_size_t, _I64, _I64],
    "llmdot_hip_release_weight": [_P, _S],
    "llmdot_hip_has_weight": [_P, _S, _PI32],
    "llmdot_hip_matmul": [_P, _P, _P, _P, _I64, _U32, _I32, _I32, _S],
    "llmdot_hip_matmul_f32": [_P, _P, _P, _P, _I64, _I32, _I32, _S],
    "llmdot_hip_rms_norm": [_P, _P, _P, _P, _I32, _F],
    "llmdot_hip_apply_rope": [_P, _P, _P, _I32, _I32, _P, _I32, _I32],
    "llmdot_hip_apply_rope_base": [_P, _P, _P, _I32, _I32, _F, _I32, _I32],
    "llmdot_hip_softmax": [_P, _P, _I32, _I32, _F],
    "llmdot_hip_silu": [_P, _P, _P, _I32],
    "llmdot_hip_layer_norm": [_P, _P, _P, _P, _P, _I32, _F],
    "llmdot_hip_gelu": [_P, _P, _P, _I32],
    "llmdot_hip_softcap": [_P, _P, _I32, _F],
    "llmdot_hip_conv1d": [_P, _P, _P, _P, _I32, _I32],
    "llmdot_hip_add": [_P, _P, _P, _P, _I32],
    "llmdot_hip_scale": [_P, _P, _F, _P, _I32],
    "llmdot_hip_mul": [_P, _P, _P, _P, _I32],
    "llmdot_hip_dequantize": [_P, _P, _P, _U32, _I32, _I32],
    "llmdot_hip_argmax": [_P, _P, _I32, _PI32],
    "llmdot_hip_sample": [_P, _P, _I32, C.POINTER(Sampling), _PI32, _I32, _F, _PI32],
    "llmdot_hip_sample_noalloc": [_P, _P, _I32, C.POINTER(Sampling), _P, _I32, _F, _P],
    "llmdot_hip_device_alloc": [_P, C.c_size_t, _PP],
    "llmdot_hip_device_free": [_P, _P],
    "llmdot_hip_memcpy_h2d": [_P, _P, _P, C.c_size_t],
    "llmdot_hip_memcpy_d2h": [_P, _P, _P, C.c_size_t],
    "llmdot_hip_synchronize": [_P],
    "llmdot_hip_gemv_device": [_P, _U32, _P, _P, _P, _I32, _I32],
    "llmdot_hip_time_gemv": [_P, _U32, _PP, _I32, _P, _P, _I32, _I32, _I32, C.POINTER(C.c_float)],
    "llmdot_hip_stream_bench": [_P, C.c_size_t, _I32, _I32, C.POINTER(C.c_float)],
    "llmdot_hip_model_create": [_P, C.POINTER(ModelDesc), _PP],
    "llmdot_hip_model_destroy": [_P],
    "llmdot_hip_model_reset": [_P],
    "llmdot_hip_decode_step": [_P, _I32, _I32, _P, _PI32],
    "llmdot_hip_prefill": [_P, _PI32, _I32, _I32, _P, _PI32],
    "llmdot_hip_generate": [_P, _PI32, _I32, _I32, _I32, _PI32, _PI32, _P],
    "llmdot_hip_generate_begin": [_P, _PI32, _I32, _I32, _I32, C.POINTER(Sampling), C.POINTER(C.c_float)],
    "llmdot_hip_generate_next": [_P, _I32, _PI32, _PI32, _PI32, _P],
    "llmdot_hip_generate_sampled": [_P, _PI32, _I32, _I32, _I32, C.POINTER(Sampling), C.POINTER(C.c_float), _PI32,
                                    _PI32, _P],
    "llmdot_hip_kv_read": [_P, _I32, _I32, _P, _P],
    "llmdot_hip_model_time_decode": [_P, _I32, _I32, _I32, _I32, C.POINTER(StepTiming)],
    "llmdot_hip_model_time_prefill": [_P, _PI32, _I32, _I32, C.POINTER(C.c_float)],
    "llmdot_hip_model_step_bytes": [_P, _I32, C.POINTER(C.c_double)],
    "llmdot_hip_model_kv_fill_random": [_P, _I32, _U64],
    "llmdot_hip_quantize": [_U32, _P, _I64, _I64, _P],
    "llmdot_hip_synth_weights": [_U32, _I64, _I64, _U64, _F, _P, _I32],
}

_lib = None
_lock = threading.Lock()


def lib() -> C.CDLL:
    """Loads libllmdot_hip.so from the package directory (raises if absent)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with dotllm_amd.build.build()")
        handle = C.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = C.c_int32
        handle.llmdot_hip_last_error.argtypes = []
        handle.llmdot_hip_last_error.restype = C.c_char_p
        _lib = handle
        return _lib


def check(rc: int) -> None:
    if rc != OK:
        msg = lib().llmdot_hip_last_error()
        raise HipError(rc, msg.decode("utf-8", "replace") if msg else "unknown error")


def ptr(a) -> C.c_void_p | None:
    """Host pointer of a C-contiguous numpy array (None for None)."""
    if a is None:
        return None
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C-contiguous")
    return C.c_void_p(a.ctypes.data)
