"""pck on MI355X: the decode hot path of proof-carrying-kernels as gfx950 HIP kernels.

The host-side numerics (`pck.fp`) and fault injection (`pck.faults`) are importable without a
GPU.  The GEMVs, the blocked checker (`pck.cuda`) and the membership check
(`pck.member.check_members`) run only through libpck_hip.so.  The reference's NumPy CPU models
(`emulate_gemv*`, `BlockedChecker`, `check_member`) are this build's test oracle and live in the
repository's `oracle/` package, outside the product.
"""

from pck.faults import flip_bit
from pck.fp import U32, U64, bf16, ceil_div, gamma, next_up, round_up_f32, sum_up, tree_height

__all__ = [
    "U32",
    "U64",
    "bf16",
    "ceil_div",
    "flip_bit",
    "gamma",
    "next_up",
    "round_up_f32",
    "sum_up",
    "tree_height",
]
