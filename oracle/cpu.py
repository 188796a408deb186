"""ctypes binding of the oracle's C restatement (oracle/cpu_qmm.c).

Test infrastructure / CPU baseline only.  Build with ``make -C oracle``.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liboracle_cpu.so")
_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} missing: run `make -C oracle`")
        lib = ctypes.CDLL(LIB_PATH)
        lib.oracle_qmm_bf16.restype = ctypes.c_int
        lib.oracle_qmm_bf16.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ]
        lib.oracle_max_threads.restype = ctypes.c_int
        _lib = lib
    return _lib


def max_threads() -> int:
    return int(load().oracle_max_threads())


def qmm_bf16(x_bits, w_q, scales_bits, biases_bits, group_size=64, bits=4, threads=0):
    """``y = x . dequant(W)^T``; bf16 bit patterns in and out, fp32 accumulate."""
    lib = load()
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    w = np.ascontiguousarray(w_q, dtype=np.uint32)
    s = np.ascontiguousarray(scales_bits, dtype=np.uint16)
    b = np.ascontiguousarray(biases_bits, dtype=np.uint16)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), dtype=np.uint16)
    rc = lib.oracle_qmm_bf16(x.ctypes.data, w.ctypes.data, s.ctypes.data, b.ctypes.data,
                             y.ctypes.data, m, k, n, int(group_size), int(bits), int(threads))
    if rc != 0:
        raise ValueError("oracle_qmm_bf16 rejected its arguments")
    return y
