"""TEST INFRASTRUCTURE — ctypes access to the oracle's scalar C models (gemv_model.c)."""

from __future__ import annotations

import ctypes
import functools

import numpy as np
from numpy.typing import NDArray

from oracle.build import LIBRARY, build

_f32p = ctypes.POINTER(ctypes.c_float)


@functools.cache
def _lib() -> ctypes.CDLL:
    if not LIBRARY.exists():
        build()
    lib = ctypes.CDLL(str(LIBRARY))
    lib.oracle_gemv_coalesced.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int64, ctypes.c_int64,
                                          ctypes.c_int, ctypes.c_int]  # fmt: skip
    lib.oracle_gemv_coalesced.restype = None
    lib.oracle_gemv_naive.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int64, ctypes.c_int64,
                                      ctypes.c_int]  # fmt: skip
    lib.oracle_gemv_naive.restype = None
    return lib


def _ptr(a: NDArray[np.float32]) -> ctypes._Pointer:  # type: ignore[type-arg]
    return a.ctypes.data_as(_f32p)


def gemv_coalesced_c(
    W: NDArray[np.float32], x: NDArray[np.float32], threads: int, vec: int = 8
) -> NDArray[np.float32]:
    """The coalesced tree computed by the scalar C model (all host cores over rows)."""
    W = np.ascontiguousarray(W, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, n = W.shape
    y = np.empty(m, dtype=np.float32)
    _lib().oracle_gemv_coalesced(_ptr(W), _ptr(x), _ptr(y), m, n, threads, vec)
    return y


def gemv_naive_c(W: NDArray[np.float32], x: NDArray[np.float32], threads: int) -> NDArray[np.float32]:
    """The naive tree computed by the scalar C model."""
    W = np.ascontiguousarray(W, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, n = W.shape
    y = np.empty(m, dtype=np.float32)
    _lib().oracle_gemv_naive(_ptr(W), _ptr(x), _ptr(y), m, n, threads)
    return y
