"""CPU oracle of the MLA + block-FP8 path and its neighbours (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
bench.py import this package, to check results.  The product package never does.

* ref_ops.py  - torch-CPU restatement of inference/ops.py:10-183 (the rounding
                points of the reference) and forward.py:92-94.
* truth.py    - the same maths in float64, naive and absorbed.
* ref_ffn.py  - SwiGLU, routing and the MoE block (inference/ops.py:186-257,
                forward.py:112-153).
* ref_head.py - final norm + lm_head and the nucleus rule of sample
                (forward.py:67-72, engine.py:166-186).
* fp8_ref.c   - C restatement of the e4m3fn decode and block dequant
                (bit-exact reference table), built by oracle/Makefile into _build/.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "_build", "libfp8ref.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB


def c_lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        lib = ctypes.CDLL(_LIB)
        lib.oracle_e4m3_to_f32.restype = ctypes.c_float
        lib.oracle_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        lib.oracle_fp8_block_dequant.restype = None
        lib.oracle_fp8_block_dequant.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                                 ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
        _lib = lib
    return _lib


def c_fp8_block_dequant(w_u8: np.ndarray, scale: np.ndarray, block: int = 128) -> np.ndarray:
    """Bit-exact fp32 dequant by the C restatement.  w_u8: (N, K) uint8 codes."""
    w_u8 = np.ascontiguousarray(w_u8, dtype=np.uint8)
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    N, K = w_u8.shape
    out = np.empty((N, K), dtype=np.float32)
    c_lib().oracle_fp8_block_dequant(w_u8.ctypes.data, scale.ctypes.data, N, K, block, out.ctypes.data)
    return out


def c_e4m3_table() -> np.ndarray:
    lib = c_lib()
    return np.array([lib.oracle_e4m3_to_f32(c) for c in range(256)], dtype=np.float32)
