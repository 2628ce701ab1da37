"""ctypes binding of oracle/mt19937_ref.c (test infrastructure only)."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "libmt19937_ref.so")
_lib = None


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            subprocess.check_call(["bash", os.path.join(_HERE, "build.sh")])
        _lib = ctypes.CDLL(_SO)
        _lib.oracle_mt19937_raw.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_size_t]
        _lib.oracle_mt19937_bits.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_size_t]
    return _lib


def raw(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    _load().oracle_mt19937_raw(seed & 0xFFFFFFFF, out.ctypes.data, n)
    return out


def bits(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    _load().oracle_mt19937_bits(seed & 0xFFFFFFFF, out.ctypes.data, n)
    return out
