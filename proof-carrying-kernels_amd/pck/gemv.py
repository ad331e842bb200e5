"""CPU models of the GEMV kernels' summation trees, in FP32 (reference `src/pck/gemv.py`, same
names, arguments and results).

These are the reference's executable specification of what its kernels compute, for callers
that model or audit a kernel on the host; the HIP GEMVs (`pck.cuda`) reproduce them bit for bit.
Each model lays the products out as one row of terms per (output row, lane) in the order that
lane adds them and sums it with `numpy.add.accumulate` in FP32, which rounds after every
addition in order; lanes are then combined in the kernel's tree order.  W and x hold values
whose products are exact in FP32 (BF16 x BF16, E4M3 x BF16), so only the additions round.
"""

from __future__ import annotations

import numpy as np
from numpy.typing import NDArray

from pck.fp import bf16, ceil_div

WARP = 32
"""Lanes per virtual warp of the coalesced kernel's reduction (reference `src/pck/gemv.py:10`)."""

Array = NDArray[np.float32]


def _products(W: NDArray[np.floating], x: NDArray[np.floating]) -> Array:
    m, n = W.shape
    if x.shape != (n,):
        raise ValueError(f"x has shape {x.shape}, expected ({n},)")
    return np.multiply(W, x, dtype=np.float32)


def _chain(terms: Array) -> Array:
    """Sequential FP32 sum of the last axis, starting from its first term."""
    return np.add.accumulate(terms, axis=-1, dtype=np.float32)[..., -1]


def _pairwise(a: Array) -> Array:
    """Neighbour-pair tree over the last axis (a power of two): ((a0 + a1) + (a2 + a3)) + ..."""
    while a.shape[-1] > 1:
        a = np.add(a[..., 0::2], a[..., 1::2], dtype=np.float32)
    return a[..., 0]


def halving_sum(a: Array) -> Array:
    """Reduce the last axis (a power of two) by halving, a[i] += a[i + len / 2], the order of a
    shuffle-down reduction with offsets len / 2, ..., 1 (reference `src/pck/gemv.py:60-68`)."""
    a = np.asarray(a, dtype=np.float32)
    while a.shape[-1] > 1:
        half = a.shape[-1] // 2
        a = np.add(a[..., :half], a[..., half:], dtype=np.float32)
    return a[..., 0]


def emulate_gemv(
    W: NDArray[np.float32],
    x: NDArray[np.float32],
    threads: int,
    *,
    acc_bf16: bool = False,
    partial_bf16: bool = False,
    drop_tail: int = 0,
) -> Array:
    """y = W x in the naive kernel's order (reference `src/pck/gemv.py:14-57`): thread t sums a
    contiguous chunk of ceil(n / threads) products in column order (columns past n are +0),
    then neighbouring threads' sums are added pairwise.

    Planted shortcuts (each breaks the accuracy contract): ``acc_bf16`` rounds the running
    per-thread sum to BF16 after every addition, ``partial_bf16`` rounds each thread's sum to
    BF16 before the tree, ``drop_tail`` skips the last ``drop_tail`` columns."""
    m, n = W.shape
    if threads < 1 or threads & (threads - 1):
        raise ValueError(f"threads must be a power of two, got {threads}")
    if not 0 <= drop_tail <= n:
        raise ValueError(f"drop_tail must be in [0, {n}], got {drop_tail}")
    P = _products(W, x)
    if drop_tail:
        P[:, n - drop_tail :] = 0.0
    chunk = ceil_div(n, threads)
    terms = np.zeros((m, threads * chunk), dtype=np.float32)
    terms[:, :n] = P
    terms = terms.reshape(m, threads, chunk)
    if acc_bf16:
        acc = terms[:, :, 0].copy()
        for j in range(1, chunk):
            acc = bf16(np.add(acc, terms[:, :, j], dtype=np.float32))
    else:
        acc = _chain(terms)
    if partial_bf16:
        acc = bf16(acc)
    return _pairwise(acc)


def emulate_gemv_coalesced(
    W: NDArray[np.float32], x: NDArray[np.float32], threads: int, vec: int = 8
) -> Array:
    """y = W x in the coalesced kernel's order (reference `src/pck/gemv.py:71-101`): columns go
    in vectors of ``vec`` (8 BF16 or 16 FP8 per 16-byte load); lane t owns vectors t,
    t + threads, ... and adds their products one at a time in column order (columns past n
    are +0); each 32-lane warp is reduced by halving and the warp sums by halving again."""
    m, n = W.shape
    if threads < WARP or threads & (threads - 1):
        raise ValueError(f"threads must be a power of two >= {WARP}, got {threads}")
    if vec < 1:
        raise ValueError(f"vec must be positive, got {vec}")
    P = _products(W, x)
    per_lane = ceil_div(ceil_div(n, vec), threads)
    padded = np.zeros((m, per_lane * threads * vec), dtype=np.float32)
    padded[:, :n] = P
    # column (v * threads + t) * vec + k is term v * vec + k of lane t
    terms = padded.reshape(m, per_lane, threads, vec).transpose(0, 2, 1, 3).reshape(m, threads, -1)
    lanes = _chain(terms)
    return halving_sum(halving_sum(lanes.reshape(m, threads // WARP, WARP)))


def reference_gemv(W: NDArray[np.floating], x: NDArray[np.floating]) -> NDArray[np.float64]:
    """y = W x in FP64 (reference `src/pck/gemv.py:104-106`)."""
    return np.asarray(W, dtype=np.float64) @ np.asarray(x, dtype=np.float64)


def abs_row_sums(W: NDArray[np.floating], x: NDArray[np.floating]) -> NDArray[np.float64]:
    """sum_j |W_ij x_j| per row, in FP64: what the rounding bound scales with (reference
    `src/pck/gemv.py:109-111`)."""
    return np.abs(np.asarray(W, dtype=np.float64)) @ np.abs(np.asarray(x, dtype=np.float64))


__all__ = ["WARP", "abs_row_sums", "emulate_gemv", "emulate_gemv_coalesced", "halving_sum",
           "reference_gemv"]  # fmt: skip
