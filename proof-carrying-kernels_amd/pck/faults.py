"""Fault injection on kernel outputs (reference `src/pck/faults.py:9-20`)."""

from __future__ import annotations

import numpy as np
from numpy.typing import NDArray


def flip_bit(y: NDArray[np.float32], index: int, bit: int) -> NDArray[np.float32]:
    """A copy of FP32 ``y`` with bit ``bit`` of element ``index`` inverted (0-22 mantissa,
    23-30 exponent, 31 sign)."""
    if y.dtype != np.float32:
        raise TypeError(f"flip_bit expects float32, got {y.dtype}")
    if not 0 <= bit < 32:
        raise ValueError(f"bit must be in [0, 32), got {bit}")
    out = y.copy()
    out.view(np.uint32)[index] ^= np.uint32(1 << bit)
    return out
