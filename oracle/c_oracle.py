"""ctypes binding of oracle/_build/liboracle.so (test oracle only; built by oracle/Makefile)."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
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
        p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.oracle_gguf_dequant.argtypes = [i32, p, i64, p]
        L.oracle_gguf_matvec.argtypes = [i32, p, p, i64, i64, p]
        L.oracle_mxfp4_dequant.argtypes = [p, p, i64, i64, p]
        L.oracle_mxfp4_matvec.argtypes = [p, p, p, p, i64, i64, p]
        for f in (L.oracle_gguf_dequant, L.oracle_gguf_matvec, L.oracle_mxfp4_dequant, L.oracle_mxfp4_matvec):
            f.restype = i32
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def gguf_dequant(data: np.ndarray, ggml_type: int, n_elems: int) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty(n_elems, dtype=np.float32)
    rc = lib().oracle_gguf_dequant(ggml_type, _ptr(data), n_elems, _ptr(out))
    if rc:
        raise ValueError(f"oracle_gguf_dequant rc={rc}")
    return out


def gguf_matvec(data: np.ndarray, ggml_type: int, x: np.ndarray, N: int, K: int) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(N, dtype=np.float32)
    rc = lib().oracle_gguf_matvec(ggml_type, _ptr(data), _ptr(x), N, K, _ptr(y))
    if rc:
        raise ValueError(f"oracle_gguf_matvec rc={rc}")
    return y


def mxfp4_dequant(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    N, G = scales.shape
    out = np.empty((N, G * 32), dtype=np.float32)
    rc = lib().oracle_mxfp4_dequant(_ptr(blocks), _ptr(scales), N, G * 32, _ptr(out))
    if rc:
        raise ValueError(f"oracle_mxfp4_dequant rc={rc}")
    return out


def mxfp4_matvec(blocks, scales, x, bias=None) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    N, G = scales.shape
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    y = np.empty(N, dtype=np.float32)
    rc = lib().oracle_mxfp4_matvec(_ptr(blocks), _ptr(scales), None if b is None else _ptr(b), _ptr(x), N, G * 32, _ptr(y))
    if rc:
        raise ValueError(f"oracle_mxfp4_matvec rc={rc}")
    return y
