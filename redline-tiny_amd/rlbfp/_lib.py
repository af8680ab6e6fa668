"""ctypes binding of librlbfp.so (the C ABI declared in include/rlbfp.h).

The library is built in-tree (``make -C redline-tiny_amd``) next to this package. There is no fallback: if it is
missing, every entry point raises. Pointers are raw device pointers; sizes are int64; the stream is a hipStream_t.
"""

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_PKG), "librlbfp.so")

# status codes (rlbfp.h)
RL_OK, RL_ERR_NULL, RL_ERR_SHAPE, RL_ERR_ARG, RL_ERR_ALIGN, RL_ERR_DEVICE, RL_ERR_WORKSPACE = range(7)
RL_DTYPE_F32, RL_DTYPE_BF16 = 0, 1
RL_ORDER_ROWBLOCK, RL_ORDER_A_LAYOUT, RL_ORDER_B_LAYOUT, RL_ORDER_C_ATB = 0, 1, 2, 3
RL_A_BF16, RL_A_BF16_QUANTIZE, RL_A_PACKED_ROWBLOCK, RL_A_PACKED_A_LAYOUT = 0, 1, 2, 3
RL_ACT_NONE, RL_ACT_GELU_TANH, RL_ACT_SWIGLU = 0, 1, 2
RL_GEMV_SILU = 3
RL_EP_QUANTIZE_OUT, RL_EP_WHOLE_K = 1, 2
RL_C_ROWMAJOR, RL_C_ATB = 0, 1
RL_NORM_LAYER, RL_NORM_RMS = 0, 1
RL_BRANCH_BF16, RL_BRANCH_PACKED = 0, 1
RL_MAX_GROUP = 16
RL_NOALLOC_SCRATCH_BYTES = 64 << 20

_ERRNAMES = {1: "RL_ERR_NULL", 2: "RL_ERR_SHAPE", 3: "RL_ERR_ARG", 4: "RL_ERR_ALIGN", 5: "RL_ERR_DEVICE",
             6: "RL_ERR_WORKSPACE"}


class RLError(RuntimeError):
    """A nonzero status from librlbfp; ``code`` is the RL_ERR_* value."""

    def __init__(self, code, msg):
        super().__init__(f"{_ERRNAMES.get(code, code)}: {msg}")
        self.code = code


class Epilogue(ctypes.Structure):
    _fields_ = [("act", ctypes.c_int32), ("flags", ctypes.c_int32), ("bias", ctypes.c_void_p),
                ("gate", ctypes.c_void_p), ("gate_split_row", ctypes.c_int64), ("residual", ctypes.c_void_p),
                ("ld_residual", ctypes.c_int64), ("packed_out", ctypes.c_void_p), ("packed_order", ctypes.c_int32),
                ("c_order", ctypes.c_int32)]


class GemmDesc(ctypes.Structure):
    _fields_ = [("A", ctypes.c_void_p), ("lda", ctypes.c_int64), ("B_packed", ctypes.c_void_p),
                ("C", ctypes.c_void_p), ("ldc", ctypes.c_int64), ("M", ctypes.c_int64), ("N", ctypes.c_int64),
                ("K", ctypes.c_int64), ("ep", Epilogue)]


# name -> (restype, argtypes); every function the header declares
_P, _I32, _I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
SIGNATURES = {
    "rl_bfp16_quantize": (ctypes.c_int, [_P, _I32, _I64, _I64, _I64, _I32, _P, _P, _P]),
    "rl_bfp16_dequantize": (ctypes.c_int, [_P, _I32, _I64, _I64, _P, _I32, _P]),
    "rl_bfp16_gemm": (ctypes.c_int, [_P, _I32, _I64, _P, _P, _I64, _I64, _I64, _I64, ctypes.POINTER(Epilogue), _P]),
    "rl_bfp16_gemm_ws": (ctypes.c_int, [_P, _I32, _I64, _P, _P, _I64, _I64, _I64, _I64, ctypes.POINTER(Epilogue),
                                        _P, _I64, _P]),
    "rl_bfp16_gemm_workspace_bytes": (ctypes.c_int64, [_I64, _I64, _I64]),
    "rl_bfp16_gemm_workspace_size": (ctypes.c_int64, [_I32, _I64, _I64, _I64]),
    "rl_bfp16_gemm_noalloc": (ctypes.c_int, [_P, _I32, _I64, _P, _P, _I64, _I64, _I64, _I64, ctypes.POINTER(Epilogue),
                                             _P]),
    "rl_bfp16_gemm_grouped": (ctypes.c_int, [ctypes.POINTER(GemmDesc), _I32, _I32, _P]),
    "rl_bfp16_gemv": (ctypes.c_int, [_P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I32, _P]),
    "rl_ln_modulate": (ctypes.c_int, [_P, _I64, _P, _I32, _I64, _P, _I64, _I32, _P, _I64, _P, _I32, _P, _I64, _I64,
                                      _I64, _P]),
    "rl_qkv_post": (ctypes.c_int, [_P, _I64, _I64, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "rl_qkv_post_gqa": (ctypes.c_int, [_P, _I64, _I64, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "rl_attention": (ctypes.c_int, [_P, _P, _P, _I32, _I64, _I64, _I64, _P, _P, _I64, _I32, _I32, _P]),
    "rl_attention_ws": (ctypes.c_int, [_P, _P, _P, _I32, _I64, _I64, _I64, _P, _P, _I64, _I32, _I32, _P, _I64, _P]),
    "rl_attention_workspace_bytes": (ctypes.c_int64, [_I32, _I64, _I64]),
    "rl_validate_quantize": (ctypes.c_int, [_I32, _I64, _I64, _I64, _I32]),
    "rl_validate_gemm": (ctypes.c_int, [_I32, _I64, _I64, _I64, _I64, _I64, ctypes.POINTER(Epilogue)]),
    "rl_validate_gemv": (ctypes.c_int, [_I64, _I64, _I64, _I64, _I64, _I32]),
    "rl_validate_ln": (ctypes.c_int, [_I64, _I32, _I64, _I32, _I64, _I32, _I64, _I64, _I64, _I64]),
    "rl_validate_qkv_post": (ctypes.c_int, [_I64, _I64, _I32]),
    "rl_validate_qkv_post_gqa": (ctypes.c_int, [_I64, _I64, _I32, _I32]),
    "rl_validate_attention": (ctypes.c_int, [_I32, _I64, _I64, _I64, _I64, _I32]),
    "rl_packed_bytes": (ctypes.c_int64, [_I64, _I64]),
    "rl_last_error": (ctypes.c_char_p, []),
    "rl_version": (ctypes.c_char_p, []),
    "rl_device_check": (ctypes.c_int, []),
}

_LIB = None


def lib():
    """The loaded library (loaded once). Raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run `make -C redline-tiny_amd`); the bfp16 path has no "
                               "fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(status):
    """Raise RLError for a nonzero status, with the library's message."""
    if status != RL_OK:
        raise RLError(status, lib().rl_last_error().decode(errors="replace"))
