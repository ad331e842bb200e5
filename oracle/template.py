"""TEST INFRASTRUCTURE — bit-exact CPU models of the agent's GEMV templates.

Restates `src/pck/agent/config.py:163-219` (the INT8 copy and the row-major model) and
`src/pck/agent/column.py:87-106` (the column-major model) of proof-carrying-kernels.  The HIP
kernels in `proof-carrying-kernels_amd/csrc/template.hip` must match these models bit for bit.
NumPy FP32 arithmetic rounds to nearest and keeps subnormals, so each model is an exact IEEE
restatement of its summation order.

How each model is pinned (tests/test_oracle_template.py):
  - `emulate` with the default knobs equals `oracle.gemv.emulate_gemv_coalesced`, which the
    C model and the reference's golden vectors pin; rows_per_block and unroll change nothing;
    every exploit knob is checked against a closed form (BF16 output = bf16 of the honest
    output, skip_tail = the honest model on W with the tail zeroed, BF16 partials = halving of
    the BF16-rounded chain sums, BF16 accumulator on two-term chains = bf16(p_t + p_{t+32})
    with the first term unrounded), small-integer sums are exact, and the honest variants
    meet the proven bound gamma_h * sum |w x| for the height the config reports;
  - `emulate_column` against an explicit per-column loop over the reference's own worked
    layout (`tests/agent/test_config.py:111-125`), against exact integer sums, against
    skipping = zeroing the skipped activations, and against the bound;
  - `quantize_rows` against its definition on hand-made groups (ties to even, an all-zero
    group, the +-127 clip, partial last groups).
"""

from __future__ import annotations

import numpy as np
from numpy.typing import NDArray

from oracle.gemv import WARP, halving_sum
from pck.agent.column import ColumnConfig
from pck.agent.config import GROUP, KernelConfig
from pck.fp import bf16, ceil_div


def quantize_rows(W: NDArray[np.float32]) -> tuple[NDArray[np.int8], NDArray[np.float32]]:
    """The INT8 copy (Wq, S) of W (reference `src/pck/agent/config.py:163-175`).

    Row i is cut into groups of ``GROUP`` columns (the last one zero-padded); a group's
    scale is its max |w| / 127 in FP32 (1 for an all-zero group) and its values are
    round-half-even(w / scale) clipped to [-127, 127].  S has shape (m, ceil(n / GROUP)).
    """
    m, n = W.shape
    groups = ceil_div(n, GROUP)
    padded = np.zeros((m, groups * GROUP), np.float32)
    padded[:, :n] = W
    by_group = padded.reshape(m, groups, GROUP)
    amax = np.abs(by_group).max(axis=2)
    scale = np.where(amax > 0, amax / np.float32(127), np.float32(1)).astype(np.float32)
    q = np.clip(np.rint(by_group / scale[:, :, None]), -127, 127).astype(np.int8)
    return np.ascontiguousarray(q.reshape(m, groups * GROUP)[:, :n]), scale


def dequantize_rows(Wq: NDArray[np.int8], S: NDArray[np.float32]) -> NDArray[np.float32]:
    """The weights an INT8 kernel multiplies x by: fl(q * scale), shape (m, n)
    (reference `src/pck/agent/config.py:178-181`)."""
    n = Wq.shape[1]
    return (Wq.astype(np.float32) * np.repeat(S, GROUP, axis=1)[:, :n]).astype(np.float32)


def emulate(
    cfg: KernelConfig | ColumnConfig, W: NDArray[np.float32], x: NDArray[np.float32]
) -> NDArray[np.float32]:
    """y = W x in the order the template instantiated with ``cfg`` computes it
    (reference `src/pck/agent/config.py:194-219`).

    Lane t of tpr lanes owns vectors t, t + tpr, ... of ``vec`` columns; its chain starts from
    its first term and adds the rest in column order (terms past n, or past the last full tile
    with ``skip_tail``, are +0), rounding to BF16 after every add with ``acc="bf16"``.  The
    chain sums (BF16-rounded with ``partials="bf16"``) are halved within 32-lane warps, then
    across warps; ``out="bf16"`` rounds y.  INT8 weights multiply the dequantized copy.
    """
    if isinstance(cfg, ColumnConfig):
        return emulate_column(cfg, W, x)
    m, n = W.shape
    if x.shape != (n,):
        raise ValueError(f"x has shape {x.shape}, expected ({n},)")
    tpr, vec = cfg.threads_per_row, cfg.vec
    if cfg.weights == "int8":
        W = dequantize_rows(*quantize_rows(W))
    per_lane = ceil_div(ceil_div(n, vec), tpr)
    width = per_lane * tpr * vec
    prod = np.zeros((m, width), np.float32)
    prod[:, :n] = (W * x).astype(np.float32)
    if cfg.skip_tail:
        prod[:, (n // (vec * tpr)) * vec * tpr :] = 0
    # column (v tpr + t) vec + k is term v vec + k of lane t
    terms = prod.reshape(m, per_lane, tpr, vec).transpose(0, 2, 1, 3).reshape(m, tpr, -1)
    acc = terms[:, :, 0].copy()
    for j in range(1, terms.shape[2]):
        acc = (acc + terms[:, :, j]).astype(np.float32)
        if cfg.acc == "bf16":
            acc = bf16(acc)
    if cfg.partials == "bf16":
        acc = bf16(acc)
    warp_sums = halving_sum(acc.reshape(m, tpr // WARP, WARP))
    y = halving_sum(warp_sums)
    return bf16(y) if cfg.out == "bf16" else y


def emulate_column(
    cfg: ColumnConfig, W: NDArray[np.float32], x: NDArray[np.float32]
) -> NDArray[np.float32]:
    """y = W x in the order of the column-major template (reference
    `src/pck/agent/column.py:87-106`).

    Grid split s owns columns [s C, (s + 1) C), C = ceil(n / splits); workgroup split k of the
    K = threads / 32 sums columns s C + k + K i for i = 0, 1, ... from +0 (skipped columns and
    columns past the range add +0).  The K sums are halved, then the ``splits`` sums.
    """
    m, n = W.shape
    if x.shape != (n,):
        raise ValueError(f"x has shape {x.shape}, expected ({n},)")
    K, S = cfg.threads // WARP, cfg.splits
    chunk = ceil_div(n, S)
    steps = ceil_div(chunk, K)
    prod = (W * x).astype(np.float32)
    if cfg.skip_below > 0:
        prod[:, np.abs(x) < np.float32(cfg.skip_below)] = 0
    by_split = np.zeros((m, S, steps * K), np.float32)
    padded = np.zeros((m, S * chunk), np.float32)
    padded[:, :n] = prod
    by_split[:, :, :chunk] = padded.reshape(m, S, chunk)
    # column s C + K i + k of the range -> [row, s, i, k]
    by_step = by_split.reshape(m, S, steps, K)
    acc = np.zeros((m, S, K), np.float32)
    for i in range(steps):
        acc = (acc + by_step[:, :, i, :]).astype(np.float32)
    return halving_sum(halving_sum(acc))
