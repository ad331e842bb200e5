"""Hypothesis strategies for GEMV problems used across the oracle and GPU tests.

A problem is BF16 weights and activations with a thread count for the summation tree.  The
row count is a multiple of ``row_multiple`` (whole checker blocks); the column count is drawn
from shape classes that exercise different code paths: exact multiples of the 8-column
vectors, ragged counts, counts below one vector, and long rows.  Values come from families
that stress different properties of a summation order: typical weights and activations, heavy
tails, a wide spread of exponents (cancellation and absorption), and exact small integers
(where every order gives the same sum).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
from hypothesis import strategies as st
from numpy.typing import NDArray

from pck.fp import bf16


@dataclass
class Problem:
    W: NDArray[np.float32]
    x: NDArray[np.float32]
    threads: int


FAMILIES = ("normal", "heavy_tail", "wide_exponents", "small_integers")


def _values(rng: np.random.Generator, family: str, shape: tuple[int, ...], scale: float) -> NDArray[np.float64]:
    if family == "normal":
        return rng.standard_normal(shape) * scale
    if family == "heavy_tail":
        return rng.standard_cauchy(shape) * scale
    if family == "wide_exponents":
        return rng.choice([-1.0, 1.0], shape) * 2.0 ** rng.uniform(-24, 24, shape)
    return rng.integers(-6, 7, shape).astype(np.float64)


@st.composite
def gemv_problems(
    draw: st.DrawFn, max_rows: int = 64, max_cols: int = 300, row_multiple: int = 1
) -> Problem:
    rows = row_multiple * draw(st.integers(1, max(1, max_rows // row_multiple)))
    kind = draw(st.sampled_from(["vectors", "ragged", "short", "long"]))
    if kind == "vectors":
        cols = 8 * draw(st.integers(1, max(1, max_cols // 8)))
    elif kind == "short":
        cols = draw(st.integers(1, min(7, max_cols)))
    elif kind == "long":
        cols = draw(st.integers(max(1, max_cols // 2), max_cols))
    else:
        cols = draw(st.integers(1, max_cols))
    family = draw(st.sampled_from(FAMILIES))
    rng = np.random.default_rng(draw(st.integers(0, 2**32 - 1)))
    W = bf16(_values(rng, family, (rows, cols), 0.02))
    x = bf16(_values(rng, family, (cols,), 1.0))
    threads = draw(st.sampled_from([1, 2, 4, 8, 16, 32, 64]))
    return Problem(W=W, x=x, threads=threads)
