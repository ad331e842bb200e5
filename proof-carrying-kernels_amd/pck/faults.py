"""Fault injection on kernel outputs and samplers (reference `src/pck/faults.py:9-42`)."""

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


def sharded_topk(
    logits: NDArray[np.float32], k: int, shards: int, per_shard: int
) -> NDArray[np.int64]:
    """An approximate top-k that can return the wrong set (reference `src/pck/faults.py:23-42`):
    the ``per_shard`` largest logits of each of ``shards`` contiguous shards
    (`numpy.array_split`), then the k largest of those, ties to the lower index.  Exact when
    ``per_shard >= k``; misses top-k logits that cluster in one shard otherwise."""
    a = np.asarray(logits, dtype=np.float32)
    if not 1 <= k <= a.size or shards < 1 or per_shard < 1:
        raise ValueError("need 1 <= k <= len(logits), shards >= 1 and per_shard >= 1")

    def best(idx: NDArray[np.int64], count: int) -> NDArray[np.int64]:
        return idx[np.lexsort((idx, -a[idx].astype(np.float64)))[:count]]

    pool = np.concatenate(
        [best(idx, per_shard) for idx in np.array_split(np.arange(a.size), shards) if idx.size]
    )
    return best(pool, k).astype(np.int64)

