"""pck on MI355X: the decode hot path of proof-carrying-kernels as gfx950 HIP kernels.

The GEMVs, the blocked checker (`pck.cuda`) and the membership check
(`pck.member.check_members`) run only through libpck_hip.so: there is no CPU fallback.  The
host-side numerics (`pck.fp`), fault injection (`pck.faults`) and the reference's CPU models of
the kernels (`pck.gemv`, `pck.checker`, `pck.sampling`, `pck.member.check_member`), which
describe what the kernels compute, are importable without a GPU.
"""

from pck.checker import BlockedChecker
from pck.faults import flip_bit
from pck.fp import U32, U64, bf16, ceil_div, gamma, next_up, round_up_f32, sum_up, tree_height
from pck.gemv import WARP, abs_row_sums, emulate_gemv, emulate_gemv_coalesced, reference_gemv

__all__ = [
    "U32",
    "U64",
    "WARP",
    "BlockedChecker",
    "abs_row_sums",
    "bf16",
    "ceil_div",
    "emulate_gemv",
    "emulate_gemv_coalesced",
    "flip_bit",
    "gamma",
    "next_up",
    "reference_gemv",
    "round_up_f32",
    "sum_up",
    "tree_height",
]
