"""TEST INFRASTRUCTURE — bit-faithful CPU models of the GEMV summation trees.

Restates `src/pck/gemv.py` of proof-carrying-kernels.  The HIP kernels in
`proof-carrying-kernels_amd/csrc/gemv.hip` must match these models bit for bit, which pins
their rounding-error bound (tree height) exactly.  All arithmetic is NumPy FP32 with
round-to-nearest; products of BF16 (or E4M3) and BF16 values are exact in FP32 barring
underflow, and NumPy does not flush subnormals, so the models are exact IEEE restatements.
"""

from __future__ import annotations

import numpy as np
from numpy.typing import NDArray

from pck.fp import bf16, ceil_div

WARP = 32
"""Lanes per virtual warp of the summation tree (reference `src/pck/gemv.py:10`)."""


def emulate_gemv(
    W: NDArray[np.float32],
    x: NDArray[np.float32],
    threads: int,
    *,
    acc_bf16: bool = False,
    partial_bf16: bool = False,
    drop_tail: int = 0,
) -> NDArray[np.float32]:
    """y = W x in the order of the naive kernel (reference `src/pck/gemv.py:14-57`).

    Lane t sums the contiguous chunk [t c, (t + 1) c), c = ceil(n / threads), starting from
    its first product (columns past n are +0), then a pairwise tree joins neighbouring lanes:
    at stride s, lane t (t % 2s == 0) adds lane t + s.

    The switches plant the reference's shortcuts, each of which breaks the accuracy spec:
    ``acc_bf16`` rounds the running sum to BF16 after every add, ``partial_bf16`` rounds each
    lane's chain sum to BF16, ``drop_tail`` skips the last ``drop_tail`` columns.
    """
    m, n = W.shape
    if x.shape != (n,):
        raise ValueError(f"x has shape {x.shape}, expected ({n},)")
    if threads < 1 or threads & (threads - 1):
        raise ValueError(f"threads must be a power of two, got {threads}")
    if not 0 <= drop_tail <= n:
        raise ValueError(f"drop_tail must be in [0, {n}], got {drop_tail}")
    chunk = ceil_div(n, threads)

    prod = (W * x).astype(np.float32)
    if drop_tail:
        prod[:, n - drop_tail :] = 0
    lanes = np.zeros((m, threads * chunk), dtype=np.float32)
    lanes[:, :n] = prod
    lanes = lanes.reshape(m, threads, chunk)

    acc = lanes[:, :, 0].copy()
    for j in range(1, chunk):
        acc = (acc + lanes[:, :, j]).astype(np.float32)
        if acc_bf16:
            acc = bf16(acc)
    if partial_bf16:
        acc = bf16(acc)
    # Pairwise tree: neighbours (2i, 2i + 1) at every level, i.e. stride 1, 2, 4, ...
    while acc.shape[1] > 1:
        acc = (acc[:, 0::2] + acc[:, 1::2]).astype(np.float32)
    return acc[:, 0]


def halving_sum(a: NDArray[np.float32]) -> NDArray[np.float32]:
    """Reduce the last axis (a power of two) by halving: a[i] += a[i + len / 2].

    Reference `src/pck/gemv.py:60-68`; the order of a shuffle-down (or xor-butterfly)
    reduction, read at lane 0.
    """
    while a.shape[-1] > 1:
        half = a.shape[-1] // 2
        a = (a[..., :half] + a[..., half:]).astype(np.float32)
    return a[..., 0]


def chain_sums_coalesced(
    W: NDArray[np.float32], x: NDArray[np.float32], threads: int, vec: int
) -> NDArray[np.float32]:
    """Per-lane chain sums (m, threads) of the coalesced tree, before any reduction.

    Lane t owns vectors t, t + threads, t + 2 threads, ... of ``vec`` columns each
    (reference `src/pck/gemv.py:71-94`) and adds their products one at a time in column
    order, starting from the first product; columns past n contribute +0.
    """
    m, n = W.shape
    per_lane = ceil_div(ceil_div(n, vec), threads)
    width = per_lane * threads * vec
    prod = np.zeros((m, width), dtype=np.float32)
    prod[:, :n] = (W * x).astype(np.float32)
    # column (v * threads + t) * vec + k  ->  term v * vec + k of lane t
    terms = prod.reshape(m, per_lane, threads, vec).transpose(0, 2, 1, 3)
    terms = terms.reshape(m, threads, per_lane * vec)
    acc = terms[:, :, 0].copy()
    for j in range(1, per_lane * vec):
        acc = (acc + terms[:, :, j]).astype(np.float32)
    return acc


def emulate_gemv_coalesced(
    W: NDArray[np.float32], x: NDArray[np.float32], threads: int, vec: int = 8
) -> NDArray[np.float32]:
    """y = W x in the order of the coalesced kernel (reference `src/pck/gemv.py:71-101`).

    Chain sums (`chain_sums_coalesced`), then halving within each virtual warp of 32 lanes,
    then halving across the threads / 32 warp sums.  Tree height `tree_height(n, threads,
    vec)`.
    """
    m, n = W.shape
    if x.shape != (n,):
        raise ValueError(f"x has shape {x.shape}, expected ({n},)")
    if threads < WARP or threads & (threads - 1):
        raise ValueError(f"threads must be a power of two >= {WARP}, got {threads}")
    if vec < 1:
        raise ValueError(f"vec must be positive, got {vec}")
    acc = chain_sums_coalesced(W, x, threads, vec)
    warp_sums = halving_sum(acc.reshape(m, threads // WARP, WARP))
    return halving_sum(warp_sums)


def reference_gemv(W: NDArray[np.floating], x: NDArray[np.floating]) -> NDArray[np.float64]:
    """FP64 y = W x (reference `src/pck/gemv.py:104-106`); its own error, about n 2^-53
    relative, is negligible beside the FP32 bounds it is compared with."""
    return W.astype(np.float64) @ x.astype(np.float64)


def abs_row_sums(W: NDArray[np.floating], x: NDArray[np.floating]) -> NDArray[np.float64]:
    """Per-row sum_j |W_ij x_j| (reference `src/pck/gemv.py:109-111`), the scale of the
    proven per-row bound |y - Wx| <= gamma_h sum_j |W_ij x_j|."""
    return np.abs(W).astype(np.float64) @ np.abs(x).astype(np.float64)


def e4m3_values() -> NDArray[np.float32]:
    """The 256 OCP E4M3FN codes decoded to FP32 (NaN for 0x7F and 0xFF).

    Decoded from the format's definition (bias 7, 3 mantissa bits, subnormals at exponent
    field 0, no infinities), independently of any library cast; the FP8 GEMV's products use
    these values.
    """
    out = np.empty(256, dtype=np.float32)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exp = (code >> 3) & 0xF
        man = code & 0x7
        if exp == 0xF and man == 0x7:
            out[code] = np.nan
        elif exp == 0:
            out[code] = sign * man * 2.0**-9
        else:
            out[code] = sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)
    return out
