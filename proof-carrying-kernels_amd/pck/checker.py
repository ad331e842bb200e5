"""The CPU blocked checker (reference `src/pck/checker.py`, same names, arguments and verdicts).

For every block beta of ``block`` output rows and secret signs r in {-1, +1}^block:

    rho = (r^T W_beta) . x - r . y_beta                        in FP64
    tau = (gamma_h + u) (a_beta . |x|) + eps(rho's rounding)   every part rounded up

with c = r^T W_beta rounded to FP32 as the GPU bank stores it and a_beta = sum_{i in beta} |W_i|
bounded above in FP32.  A block passes only if its outputs are finite, tau is finite and
|rho| <= tau; NaN and Inf raise the alarm.  The GPU checker (`pck.cuda.GpuBlockedChecker`)
computes the same check from a stored bank.
"""

from __future__ import annotations

import numpy as np
from numpy.typing import NDArray

from pck.fp import U32, U64, gamma, next_up, round_up_f32, sum_up


class WeightBank:
    """The W-only part of the check, built once per weight matrix and block size (reference
    `src/pck/checker.py:11-24`): W in FP64 per block, and per block and column the upper bound
    a_up of sum_i |W_ij| rounded up to FP32."""

    def __init__(self, W: NDArray[np.floating], block: int) -> None:
        m, n = W.shape
        if block < 1 or m % block:
            raise ValueError(f"block={block} must be positive and divide m={m}")
        self.shape, self.block = (m, n), block
        self.W_blocks = np.asarray(W, dtype=np.float64).reshape(m // block, block, n)
        with np.errstate(over="ignore", invalid="ignore"):
            # past the FP32 range a_up is inf: tau is inf and the check fails closed
            self.a_up = round_up_f32(sum_up(np.abs(self.W_blocks).sum(axis=1), block))


class BlockedChecker:
    """One random-sign checksum per block of ``block`` rows of y = W x (reference
    `src/pck/checker.py:27-99`); ``height`` is the summation tree height of the kernel under
    check (`pck.fp.tree_height`)."""

    def __init__(
        self,
        W: NDArray[np.floating],
        x: NDArray[np.floating],
        block: int,
        height: int,
        bank: WeightBank | None = None,
    ) -> None:
        m, n = W.shape
        if x.shape != (n,):
            raise ValueError(f"x has shape {x.shape}, expected ({n},)")
        if bank is None:
            bank = WeightBank(W, block)
        elif bank.shape != (m, n) or bank.block != block:
            raise ValueError("the weight bank was built for another W or block")
        self.m, self.n, self.block = m, n, block
        self.num_blocks = m // block
        self.W_blocks = bank.W_blocks
        self.x = np.asarray(x, dtype=np.float64)
        with np.errstate(over="ignore", invalid="ignore"):
            self.abs_bound: NDArray[np.float64] = sum_up(bank.a_up @ np.abs(self.x), n)
        """An upper bound of a_beta . |x| per block."""
        self.gamma_h = gamma(height)
        self.coef = next_up(next_up(self.gamma_h) + U32)
        """gamma_h + u32, rounded up."""

    @property
    def tau_base(self) -> NDArray[np.float64]:
        """(gamma_h + u) (a_beta . |x|) per block, rounded up: the part of tau that does not
        depend on y or the signs."""
        with np.errstate(over="ignore", invalid="ignore"):
            return np.nextafter(self.coef * self.abs_bound, np.inf)

    def _check(self, yb: NDArray[np.float64], r: NDArray[np.float64]) -> NDArray[np.bool_]:
        """Pass / fail per block for one draw of signs r (num_blocks, block)."""
        c = np.einsum("kb,kbn->kn", r, self.W_blocks).astype(np.float32).astype(np.float64)
        with np.errstate(invalid="ignore", over="ignore"):
            rho = c @ self.x - (r * yb).sum(axis=1)
            magnitude = sum_up(np.abs(c) @ np.abs(self.x), self.n) + sum_up(
                np.abs(yb).sum(axis=1), self.block
            )
            eps = np.nextafter(next_up(gamma(self.n + self.block + 1, U64)) * magnitude, np.inf)
            tau = np.nextafter(self.tau_base + eps, np.inf)
            return np.isfinite(tau) & (np.abs(rho) <= tau)  # NaN compares false

    def verdict(
        self, y: NDArray[np.floating], rng: np.random.Generator, checks: int = 1
    ) -> NDArray[np.bool_]:
        """Per-block pass (True) or fail of output ``y`` after ``checks`` independent draws of
        signs from ``rng`` (one (num_blocks, block) draw per check, the reference's order);
        ``rng`` must be independent of how ``y`` was produced."""
        if y.shape != (self.m,):
            raise ValueError(f"y has shape {y.shape}, expected ({self.m},)")
        with np.errstate(invalid="ignore", over="ignore"):
            yb = np.asarray(y, dtype=np.float64).reshape(self.num_blocks, self.block)
        ok = np.isfinite(yb).all(axis=1)
        for _ in range(checks):
            ok &= self._check(yb, rng.choice([-1.0, 1.0], (self.num_blocks, self.block)))
        return ok


__all__ = ["BlockedChecker", "WeightBank"]
