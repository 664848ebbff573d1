"""ctypes loader for oracle/gemv_ref.c (test infrastructure only; see oracle/__init__.py).

The shared library is built by ``make -C oracle`` (``__graft_entry__.build()`` runs it).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_gemv.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_e4m3_lut.argtypes = [ctypes.c_void_p]
        L.oracle_gemv_fp8_seq.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 3
        L.oracle_bf16_rne.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
        _lib = L
    return _lib


def e4m3_lut() -> np.ndarray:
    out = np.empty(256, dtype=np.float32)
    lib().oracle_e4m3_lut(out.ctypes.data)
    return out


def gemv_fp8_seq(x_bits: np.ndarray, w_codes: np.ndarray, s: np.ndarray) -> np.ndarray:
    """Sequential fp32 GEMV of tests/ops/test_gemm.cu:505-513 for every row of x.
    x uint16 [M,K] (or [K]), W uint8 [N,K], s float32 [N] -> float32 [M,N] (or [N])."""
    x = np.ascontiguousarray(np.atleast_2d(x_bits), dtype=np.uint16)
    w = np.ascontiguousarray(w_codes, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    M, K = x.shape
    N = w.shape[0]
    assert w.shape[1] == K and s.shape[0] == N
    y = np.empty((M, N), dtype=np.float32)
    lib().oracle_gemv_fp8_seq(x.ctypes.data, w.ctypes.data, s.ctypes.data, y.ctypes.data, M, N, K)
    return y[0] if np.asarray(x_bits).ndim == 1 else y


def bf16_rne(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    lib().oracle_bf16_rne(f.ctypes.data, out.ctypes.data, f.size)
    return out
