"""TEST INFRASTRUCTURE — the CPU top-k / top-p set checker and reference samplers.

Restates `src/pck/sampling.py:38-127` of proof-carrying-kernels (the trusted CPU checker that
`check_topk_gpu` / `check_topp_gpu` mirror).  Only tests import this module; the library's
set checker (`csrc/sampling.hip`) never calls it.

A selection passes top-k when it is k distinct in-range indices and no rejected logit is
larger than a selected one (exact FP32 comparisons; ties either way; any NaN fails).  Top-p
adds minimality with FP64 softmax masses: mass(S) >= p - slack and
mass(S without its smallest logit) < p + slack, slack = next_up(tol + softmax_eps(V, zmax)),
the bounds rounded outward.
"""

from __future__ import annotations

import math

import numpy as np
from numpy.typing import ArrayLike, NDArray

from pck.fp import next_up, softmax_eps


def as_logits(logits: ArrayLike) -> NDArray[np.float32]:
    """Non-empty 1-D FP32 logits (reference `sampling.py:31-35`)."""
    a = np.asarray(logits, dtype=np.float32)
    if a.ndim != 1 or a.size == 0:
        raise ValueError("logits must be a non-empty 1-D array")
    return a


def _descending(a: NDArray[np.float32]) -> NDArray[np.int64]:
    """Indices by decreasing logit, ties by increasing index."""
    return np.lexsort((np.arange(a.size), -a.astype(np.float64))).astype(np.int64)


def topk_reference(logits: ArrayLike, k: int) -> NDArray[np.int64]:
    """The k largest logits, ties to the lower index (reference `sampling.py:38-44`)."""
    a = as_logits(logits)
    if not 1 <= k <= a.size:
        raise ValueError(f"k must be in [1, {a.size}], got {k}")
    return _descending(a)[:k]


def softmax64(logits: ArrayLike, temperature: float = 1.0) -> NDArray[np.float64]:
    """FP64 softmax of logits / temperature (reference `sampling.py:47-54`)."""
    if not temperature > 0:
        raise ValueError(f"temperature must be positive, got {temperature}")
    z = as_logits(logits).astype(np.float64) / temperature
    e = np.exp(z - z.max())
    return e / e.sum()


def topp_reference(logits: ArrayLike, p: float, temperature: float = 1.0) -> NDArray[np.int64]:
    """The shortest descending prefix whose FP64 mass reaches p (reference
    `sampling.py:57-66`)."""
    if not 0 < p <= 1:
        raise ValueError(f"p must be in (0, 1], got {p}")
    a = as_logits(logits)
    order = _descending(a)
    running = np.cumsum(softmax64(a, temperature)[order])
    count = min(int(np.searchsorted(running, p)) + 1, a.size)
    return order[:count]


def selection_mask(size: int, selected: ArrayLike) -> NDArray[np.bool_] | None:
    """Membership mask of a selection, or None when it is not a non-empty 1-D set of distinct
    in-range integer indices (reference `sampling.py:69-79`)."""
    s = np.asarray(selected)
    if s.ndim != 1 or s.size == 0 or not np.issubdtype(s.dtype, np.integer):
        return None
    if s.min() < 0 or s.max() >= size or np.unique(s).size != s.size:
        return None
    mask = np.zeros(size, dtype=bool)
    mask[s] = True
    return mask


def is_prefix(a: NDArray[np.float32], mask: NDArray[np.bool_]) -> bool:
    """No NaN, and min over the selected >= max over the rejected (reference
    `sampling.py:82-88`)."""
    if np.isnan(a).any():
        return False
    return bool(mask.all() or a[mask].min() >= a[~mask].max())


def check_topk(logits: ArrayLike, selected: ArrayLike, k: int) -> bool:
    """Reference `sampling.py:91-95`."""
    a = as_logits(logits)
    mask = selection_mask(a.size, selected)
    return mask is not None and int(mask.sum()) == k and is_prefix(a, mask)


def check_topp(
    logits: ArrayLike, selected: ArrayLike, p: float, temperature: float = 1.0, tol: float = 1e-6
) -> bool:
    """Reference `sampling.py:98-122`: prefix, then FP64 masses against p -/+ slack."""
    if not 0 < p <= 1:
        raise ValueError(f"p must be in (0, 1], got {p}")
    if tol < 0:
        raise ValueError(f"tol must be non-negative, got {tol}")
    a = as_logits(logits)
    mask = selection_mask(a.size, selected)
    if mask is None or not is_prefix(a, mask):
        return False
    probs = softmax64(a, temperature)
    mass = float(probs[mask].sum())
    chosen = np.flatnonzero(mask)
    without = mass - float(probs[chosen[np.argmin(a[chosen])]])
    finite = a[np.isfinite(a)]
    zmax = 0.0 if temperature == 1.0 else float(np.abs(finite / temperature).max(initial=0.0))
    slack = next_up(tol + softmax_eps(a.size, zmax))
    return mass >= math.nextafter(p - slack, -math.inf) and without < next_up(p + slack)


def check_sampled(token: int, selected: ArrayLike) -> bool:
    """Reference `sampling.py:125-127`."""
    return bool(np.isin(token, np.asarray(selected)))
