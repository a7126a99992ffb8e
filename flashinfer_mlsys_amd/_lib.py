"""ctypes binding of libmoe_mi355x.so (declarations in include/moe_fp8.h).

The library is loaded on first use. There is no fallback: if the shared
library is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmoe_mi355x.so")

MOE_OK = 0
MOE_ERR_NULL = -1
MOE_ERR_SIZE = -2
MOE_ERR_ALIGN = -3
MOE_ERR_WORKSPACE = -4
MOE_ERR_HIP = -5
MOE_ERR_ARG = -6
MOE_ERR_NOALLOC_SIZE = -7
MOE_FP8_NOALLOC_MAX_TOKENS = 64
MOE_FP8_DECODE_MAX_TOKENS = 96  # MOE_SHAPE_AUTO: the decode kernels up to here
MOE_FP8_MAX_TOKENS = 1 << 20      # the forward entry points
MOE_FP8_MAX_TAP_TOKENS = 1 << 17  # every other entry point
MOE_FP8_CHUNK_TOKENS = 1 << 14
MOE_FP8_HEADER_WORDS = 128

MOE_SHAPE_AUTO = 0
MOE_SHAPE_PREFILL = 1

# Every symbol the header declares, with its ctypes signature.
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
SIGNATURES = {
    "moe_fp8_workspace_size": (ctypes.c_size_t, [_I64]),
    "moe_fp8_forward": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, ctypes.c_double, _P, _P,
                                       ctypes.c_size_t, _P]),
    "moe_fp8_forward_noalloc": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, ctypes.c_double, _P,
                                               _P]),
    "moe_fp8_forward_shape": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64,
                                             ctypes.c_double, _P, _P, ctypes.c_size_t, _P]),
    "moe_fp8_run_stage": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64,
                                         ctypes.c_double, _P, _P, ctypes.c_size_t, _P]),
    "moe_fp8_route": (ctypes.c_int, [_P, _P, _I64, ctypes.c_double, _P, _P, _P, _P]),
    "moe_fp8_quantize_activations": (ctypes.c_int, [_P, _I64, _P, _P, _P]),
    "moe_fp8_router_logits": (ctypes.c_int, [_P, _P, _I64, _P, _P]),
    "moe_fp8_router_quantize": (ctypes.c_int, [_P, _P, _I64, _P, _P, _P, _P]),
    "moe_fp8_dispatch": (ctypes.c_int, [_P, _P, _I64, _I64, _P, ctypes.c_size_t, _P, _P, _P, _P]),
    "moe_fp8_route_dispatch": (ctypes.c_int, [ctypes.c_int, _P, _P, _I64, _I64, ctypes.c_double, _P, _P, _P,
                                              ctypes.c_size_t, _P, _P,
                                              _P, _P]),
    "moe_fp8_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "moe_fp8_last_hip_error": (ctypes.c_char_p, []),
    "moe_fp8_abi_version": (ctypes.c_int, []),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build the MI355X kernels with "
                    "`python -m flashinfer_mlsys_amd.build` (there is no fallback path)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(code: int, what: str) -> None:
    if code == MOE_OK:
        return
    lib = load()
    msg = lib.moe_fp8_strerror(code).decode()
    if code == MOE_ERR_HIP:
        msg += ": " + lib.moe_fp8_last_hip_error().decode()
    raise RuntimeError(f"{what} failed ({code}): {msg}")
