"""ctypes binding of ``libnnq.so`` (the C ABI declared in ``include/nnq.h``).

Loading fails loudly: there is no CPU fallback for any compute entry point.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnnq.so")

c_void_p = ctypes.c_void_p
c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_sz = ctypes.c_size_t
c_float = ctypes.c_float
c_u64 = ctypes.c_uint64
c_double = ctypes.c_double


class Sampling(ctypes.Structure):
    """nnq_sampling (include/nnq.h)."""
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_int32), ("use_top_p", ctypes.c_int32),
                ("top_p", ctypes.c_float), ("repetition_penalty", ctypes.c_float),
                ("frequency_penalty", ctypes.c_float), ("seed", ctypes.c_uint64)]

# name -> (restype, argtypes); every symbol declared in include/nnq.h
SIGNATURES = {
    "nnq_device_count": (c_int, [ctypes.POINTER(c_int)]),
    "nnq_init": (c_int, [c_int]),
    "nnq_last_error": (ctypes.c_char_p, []),
    "nnq_weight_create": (c_int, [c_int, c_int, c_void_p, c_sz, c_i64, c_i64, ctypes.POINTER(c_void_p)]),
    "nnq_weight_destroy": (c_int, [c_void_p]),
    "nnq_weight_info": (c_int, [c_void_p, ctypes.POINTER(c_int), ctypes.POINTER(c_int), ctypes.POINTER(c_i64),
                                ctypes.POINTER(c_i64), ctypes.POINTER(c_sz)]),
    "nnq_dequant": (c_int, [c_void_p, c_void_p, c_void_p]),
    "nnq_linear": (c_int, [c_void_p, c_void_p, c_int, c_i64, c_i64, c_void_p, c_i64, c_void_p, c_int, c_void_p]),
    "nnq_argmax_f32": (c_int, [c_void_p, c_i64, c_void_p, c_void_p, c_void_p]),
    "nnq_linear_argmax": (c_int, [c_void_p, c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_void_p, c_void_p,
                                  c_void_p]),
    "nnq_moe_create": (c_int, [c_i64, c_i64, c_i64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                               ctypes.POINTER(c_void_p)]),
    "nnq_moe_destroy": (c_int, [c_void_p]),
    "nnq_moe_forward": (c_int, [c_void_p, c_void_p, c_int, c_i64, c_void_p, c_int, c_float, c_void_p, c_void_p,
                                c_void_p, c_void_p]),
    "nnq_moe_dequant_expert": (c_int, [c_void_p, c_i64, c_void_p, c_void_p, c_void_p]),
    "nnq_router_create": (c_int, [c_i64, c_i64, c_void_p, c_void_p, ctypes.POINTER(c_void_p)]),
    "nnq_router_destroy": (c_int, [c_void_p]),
    "nnq_router_logits": (c_int, [c_void_p, c_void_p, c_int, c_i64, c_void_p, c_void_p]),
    "nnq_moe_block_forward": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_i64, c_int, c_float, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_void_p]),
    "nnq_mlp_create": (c_int, [c_int, c_int, c_void_p, c_void_p, c_sz, c_int, c_int, c_void_p, c_sz, c_i64, c_i64,
                               ctypes.POINTER(c_void_p)]),
    "nnq_mlp_destroy": (c_int, [c_void_p]),
    "nnq_mlp_forward": (c_int, [c_void_p, c_void_p, c_int, c_i64, c_i64, c_void_p, c_int, c_void_p, c_void_p]),
    "nnq_sample_token": (c_int, [c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_void_p, c_void_p]),
    "nnq_linear_sample": (c_int, [c_void_p, c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_void_p, c_i64, c_void_p,
                                  c_void_p, c_void_p]),
    "nnq_moe_create_ocp": (c_int, [c_i64, c_i64, c_i64, c_void_p, c_void_p, c_void_p, c_void_p,
                                   ctypes.POINTER(c_void_p)]),
    "nnq_dequant_mxfp4_ocp": (c_int, [c_void_p, c_i64, c_void_p, c_void_p]),
    "nnq_quantize_mxfp4_ocp": (c_int, [c_void_p, c_sz, c_void_p]),
    "nnq_release_workspace": (c_int, [c_void_p]),
    "nnq_release_capture_workspaces": (c_int, []),
    "nnq_linear_sample_noalloc": (c_int, [c_void_p, c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_void_p, c_i64,
                                          c_void_p, c_void_p, c_void_p]),
    "nnq_gguf_open": (c_int, [ctypes.c_char_p, ctypes.POINTER(c_void_p)]),
    "nnq_gguf_close": (c_int, [c_void_p]),
    "nnq_gguf_info": (c_int, [c_void_p, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(c_i64),
                              ctypes.POINTER(c_i64), ctypes.POINTER(c_u64)]),
    "nnq_gguf_tensor_info": (c_int, [c_void_p, c_i64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int32),
                                     ctypes.POINTER(c_u64), ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(c_u64),
                                     ctypes.POINTER(c_u64)]),
    "nnq_gguf_tensor_data": (c_int, [c_void_p, ctypes.c_char_p, ctypes.POINTER(c_void_p), ctypes.POINTER(c_u64)]),
    "nnq_gguf_metadata": (c_int, [c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(c_u64),
                                  ctypes.POINTER(c_i64), ctypes.POINTER(c_double), ctypes.POINTER(ctypes.c_char_p),
                                  ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(c_u64)]),
    "nnq_gguf_weight_create": (c_int, [c_void_p, ctypes.c_char_p, c_int, c_int, ctypes.POINTER(c_void_p)]),
    "nnq_quantize_q4_k": (c_int, [c_void_p, c_sz, c_void_p]),
    "nnq_quantize_mxfp4": (c_int, [c_void_p, c_sz, c_void_p, c_void_p]),
    "nnq_quantize_q8_0": (c_int, [c_void_p, c_sz, c_void_p]),
    "nnq_quantize_q6_k": (c_int, [c_void_p, c_sz, c_void_p]),
    "nnq_synth_normal": (c_int, [c_u64, c_u64, c_sz, c_double, c_void_p]),
}

# status codes (nnq_status)
OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_SHAPE_MISMATCH = 2
ERR_WRONG_FORMAT = 3
ERR_NOT_QUANTIZED = 4
ERR_WEIGHT_RANK = 5
ERR_BIAS_MISMATCH = 6
ERR_DATA_LENGTH = 7
ERR_INVALID_SHAPE = 8
ERR_NON_FINITE = 9
ERR_NO_DEVICE = 10
ERR_OUT_OF_MEMORY = 11
ERR_DISPATCH_FAILED = 12
ERR_UNSUPPORTED = 13

_lib = None


def load():
    """Load libnnq.so and attach signatures; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"nnq native library not built: {LIB_PATH} is missing "
                               "(run `python -m nn_amd.build`); there is no fallback path")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error() -> str:
    return load().nnq_last_error().decode(errors="replace")
