"""ctypes binding of oracle/bfp16_ref.c (oracle; test infrastructure only). Build with ``make -C oracle``."""

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "libbfp16_ref.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built: run `make -C oracle`")
        L = ctypes.CDLL(path)
        for name in ("rl_ref_to_bfp16", "rl_ref_to_bfp16_truncate"):
            getattr(L, name).argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        L.rl_ref_from_bfp16.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        _LIB = L
    return _LIB


def to_bfp16(x, truncate=False):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert x.size % 8 == 0
    out = np.empty(x.size // 8 * 9, dtype=np.uint8)
    fn = lib().rl_ref_to_bfp16_truncate if truncate else lib().rl_ref_to_bfp16
    fn(x.ctypes.data, x.size // 8, out.ctypes.data)
    return out


def from_bfp16(raw):
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    assert raw.size % 9 == 0
    out = np.empty(raw.size // 9 * 8, dtype=np.float32)
    lib().rl_ref_from_bfp16(raw.ctypes.data, raw.size // 9, out.ctypes.data)
    return out
