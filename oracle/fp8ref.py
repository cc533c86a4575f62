"""ctypes loader for oracle/fp8_ref.c — TEST INFRASTRUCTURE ONLY."""
from __future__ import annotations

import ctypes
from ctypes import c_int64, c_void_p

import numpy as np

from . import build as _build

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _build.LIB.exists():
            _build.build()
        h = ctypes.CDLL(str(_build.LIB))
        h.fp8ref_decode.restype = ctypes.c_double
        h.fp8ref_decode.argtypes = [ctypes.c_uint8]
        h.fp8ref_encode.restype = ctypes.c_uint8
        h.fp8ref_encode.argtypes = [ctypes.c_float]
        h.fp8ref_per_token_quant.argtypes = [c_void_p, c_int64, c_int64, c_void_p, c_void_p]
        h.fp8ref_group_quant.argtypes = [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p]
        h.fp8ref_encode_array.argtypes = [c_void_p, c_int64, c_void_p]
        _lib = h
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def decode(code: int) -> float:
    return lib().fp8ref_decode(code)


def encode_array(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(v.shape, dtype=np.uint8)
    lib().fp8ref_encode_array(_ptr(v), v.size, _ptr(out))
    return out


def per_token_quant(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """x: fp32 [M, K] -> (q uint8 [M, K], s fp32 [M])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    q = np.empty((M, K), dtype=np.uint8)
    s = np.empty((M,), dtype=np.float32)
    lib().fp8ref_per_token_quant(_ptr(x), M, K, _ptr(q), _ptr(s))
    return q, s


def group_quant(x: np.ndarray, group: int) -> tuple[np.ndarray, np.ndarray]:
    """x: fp32 [M, K] -> (q uint8 [M, K], s fp32 [M, K/group])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    q = np.empty((M, K), dtype=np.uint8)
    s = np.empty((M, K // group), dtype=np.float32)
    lib().fp8ref_group_quant(_ptr(x), M, K, group, _ptr(q), _ptr(s))
    return q, s
