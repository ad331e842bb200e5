"""Host-side floating-point constants for the GEMV, checker and membership paths.

Everything here is scalar or elementwise host arithmetic that the HIP paths need before a
launch (tree heights, Higham's gamma_k, outward-rounded coefficients).  The formulas follow
`src/pck/fp.py` of proof-carrying-kernels line for line in meaning; the IEEE-double operation
order is kept so that every constant has the same bits as the reference's.
"""

from __future__ import annotations

import math

import numpy as np
from numpy.typing import ArrayLike, NDArray

U32: float = 2.0**-24
"""FP32 unit roundoff under round-to-nearest (reference `src/pck/fp.py:10`)."""

U64: float = 2.0**-53
"""FP64 unit roundoff under round-to-nearest (reference `src/pck/fp.py:13`)."""

_LOW16 = np.uint32(0xFFFF)
_HIGH16 = np.uint32(0xFFFF0000)


def bf16(a: ArrayLike) -> NDArray[np.float32]:
    """FP32 values rounded to the nearest BF16 (ties to even), returned as FP32.

    Reference `src/pck/fp.py:17-28`.  Rounding adds 0x7FFF plus the lowest kept bit to the
    raw bits and clears the low half; overflow carries into +/-Inf as BF16 hardware does.
    NaN inputs stay NaN (the carry could otherwise turn a NaN payload into Inf).
    """
    out = np.array(a, dtype=np.float32, copy=True)
    was_nan = np.isnan(out)
    raw = out.view(np.uint32)
    raw += np.uint32(0x7FFF) + ((raw >> np.uint32(16)) & np.uint32(1))
    raw &= _HIGH16
    out[was_nan] = np.nan
    return out


def gamma(k: int, u: float = U32) -> float:
    """Higham's constant gamma_k = k u / (1 - k u) (reference `src/pck/fp.py:31-37`)."""
    if k < 0:
        raise ValueError(f"k must be non-negative, got {k}")
    if k * u >= 1:
        raise ValueError(f"gamma_k needs k*u < 1, got k*u = {k * u}")
    return k * u / (1 - k * u)


def round_up_f32(v: ArrayLike) -> NDArray[np.float64]:
    """Non-negative FP64 values stored as FP32, never rounded down; returned widened to FP64.

    Reference `src/pck/fp.py:40-51`.
    """
    wide = np.asarray(v, dtype=np.float64)
    if np.any(wide < 0):
        raise ValueError("round_up_f32 expects non-negative values")
    narrow = wide.astype(np.float32)
    short = narrow.astype(np.float64) < wide
    narrow[short] = np.nextafter(narrow[short], np.float32(np.inf))
    return narrow.astype(np.float64)


def next_up(v: float, steps: int = 1) -> float:
    """``v`` raised by ``steps`` FP64 ulps (reference `src/pck/fp.py:54-58`)."""
    for _ in range(steps):
        v = math.nextafter(v, math.inf)
    return v


def sum_up_factor(terms: int) -> float:
    """Multiplier that lifts a round-to-nearest FP64 sum of ``terms`` non-negative values to
    an upper bound of the exact sum: S <= s (1 + 2 gamma_terms(u64)), itself rounded up.

    Reference `src/pck/fp.py:61-66`.
    """
    return next_up(1.0 + 2.0 * gamma(max(terms, 1), U64))


def sum_up(s: ArrayLike, terms: int) -> NDArray[np.float64]:
    """Upper bounds of the exact sums whose FP64 round-to-nearest values are ``s``.

    Reference `src/pck/fp.py:69-73`: multiply by `sum_up_factor` and round the product up.
    """
    wide = np.asarray(s, dtype=np.float64)
    with np.errstate(over="ignore"):
        return np.nextafter(wide * sum_up_factor(terms), np.inf)


def softmax_eps(vocab: int, zmax: float = 0.0) -> float:
    """Bound on the error of an FP64 softmax mass over ``vocab`` logits.

    Reference `src/pck/fp.py:76-99` (derivation in its docstring): per-term error E from the
    argument rounding (u |x| + 2 zmax u), a 2-ulp ``exp`` and the FP64 sum, then the quotient
    and one subtraction.  Raises when E exceeds 0.01, where the bound stops holding.
    """
    u = U64
    v = max(vocab, 1)
    e = 1.01 * (v * u / math.e + 2.0 * zmax * u + 4.0 * u) + 1.01 * gamma(v, u)
    if not e <= 0.01:
        raise ValueError(
            f"softmax over {vocab} logits with |logit / T| up to {zmax} is too "
            "large to check in FP64"
        )
    return (2.0 * e + gamma(v + 2, u) * (1.0 + e)) / (1.0 - e) + 2.0 * u


def ceil_div(a: int, b: int) -> int:
    """ceil(a / b) for a >= 0 and b > 0."""
    return -(-a // b)


def tree_height(n: int, threads: int, vec: int = 1) -> int:
    """Height of the GEMV summation tree over ``n`` columns with ``threads`` lanes.

    Reference `src/pck/fp.py:107-124`.  A lane sums its chain sequentially (``vec`` columns
    per vector, every ``threads``-th vector; vec = 1 is one contiguous chunk per lane), then
    a binary tree of height log2(threads) joins the lanes.  The chain has
    vec * ceil(ceil(n / vec) / threads) terms, padding included.
    """
    if n < 1:
        raise ValueError(f"n must be positive, got {n}")
    if threads < 1 or threads & (threads - 1):
        raise ValueError(f"threads must be a power of two, got {threads}")
    if vec < 1:
        raise ValueError(f"vec must be positive, got {vec}")
    chain = vec * ceil_div(ceil_div(n, vec), threads)
    return (chain - 1) + threads.bit_length() - 1
