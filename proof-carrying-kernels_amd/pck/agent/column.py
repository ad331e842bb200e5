"""Knobs of the column-major GEMV template (reference `src/pck/agent/column.py:31-85`).

W is stored transposed once at weight load (``WT = W^T``, shape (n, m)), so column j of W is
the contiguous row ``WT[j]``.  A workgroup of ``threads`` lanes is K = threads / 32 column
splits of 32 lanes each; lane g of split k owns ``vec`` consecutive output rows.  The grid adds
``splits`` more splits along n: grid split s owns the contiguous columns [s C, (s + 1) C),
C = ceil(n / splits), and split k of the workgroup sums columns s C + k, s C + k + K, ... of
that range in order from +0.  The K sums are joined by halving, then the ``splits`` grid sums
by halving, so the tree height is (ceil(C / K) - 1) + log2(K splits).

``skip_below > 0`` is the planted activation-sparsity exploit: every column with
|x_j| < skip_below is skipped and its row of WT never read.
"""

from __future__ import annotations

import itertools
from dataclasses import asdict, dataclass
from typing import Literal

from pck.fp import ceil_div

WARP = 32
COL_THREADS = (32, 64, 128, 256)
COL_VECS = (2, 4, 8)
SPLITS = (1, 2, 4, 8, 16, 32, 64)
SKIP_BELOW = (0.0, 0.005, 0.01, 0.02, 0.03, 0.05, 0.1, 0.3)


@dataclass(frozen=True)
class ColumnConfig:
    threads: int = 128
    vec: int = 8
    splits: int = 32
    skip_below: float = 0.0
    layout: Literal["col"] = "col"

    def __post_init__(self) -> None:
        errors = self.validate()
        if errors:
            raise ValueError("; ".join(errors))

    def validate(self) -> list[str]:
        """Why the template cannot take this config (empty when it can)."""
        allowed = {
            "threads": COL_THREADS,
            "vec": COL_VECS,
            "splits": SPLITS,
            "skip_below": SKIP_BELOW,
            "layout": ("col",),
        }
        errors = []
        for name, values in allowed.items():
            value = getattr(self, name)
            if type(value) is not type(values[0]) or value not in values:
                errors.append(f"{name} must be one of {list(values)}, got {value!r}")
        return errors

    @property
    def out(self) -> str:
        return "fp32"

    @property
    def num_splits(self) -> int:
        """Splits of the n axis in all: K per workgroup times the grid's ``splits``."""
        return self.threads // WARP * self.splits

    def tree_height(self, n: int) -> int:
        chain = ceil_div(ceil_div(n, self.splits), self.threads // WARP)
        return chain - 1 + self.num_splits.bit_length() - 1

    def as_dict(self) -> dict[str, object]:
        return asdict(self)


def column_space() -> list[ColumnConfig]:
    """Every valid column-major config, threads slowest and skip_below fastest."""
    return [
        ColumnConfig(t, v, s, k)
        for t, v, s, k in itertools.product(COL_THREADS, COL_VECS, SPLITS, SKIP_BELOW)
    ]
