"""TEST INFRASTRUCTURE — the CPU blocked checker and an exact model of the GPU threshold.

`WeightBank` and `BlockedChecker` restate `src/pck/checker.py:11-99` of
proof-carrying-kernels (the trusted CPU checker).  `BlockedChecker.verdict_with_signs` takes
the sign vectors explicitly, so a test can give the CPU checker and the HIP checker the same
(W, x, y, r) and compare verdicts (the reference draws CPU signs per call from a NumPy
generator and GPU signs once from a torch generator, so only equal inputs can be compared).

`gpu_threshold_exact` evaluates the GPU checker's threshold formula
(`src/pck/cuda/csrc/checker_kernel.cu:176-181`) in exact rational arithmetic from the stored
bank; the HIP checker rounds every operation of it upward, so its tau must never fall below
this value and may exceed it only by the FP32 round-up slack.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
from numpy.typing import NDArray

from pck.fp import U32, U64, gamma, next_up, round_up_f32, sum_up


class WeightBank:
    """The W-only part of the CPU check: W in FP64 blocks and a_beta = sum_i |W_i| bounded
    above and rounded up to FP32 (reference `src/pck/checker.py:11-24`)."""

    def __init__(self, W: NDArray[np.floating], block: int) -> None:
        m, n = W.shape
        if block < 1 or m % block:
            raise ValueError(f"block={block} must be positive and divide m={m}")
        self.shape, self.block = (m, n), block
        self.W_blocks = W.reshape(m // block, block, n).astype(np.float64)
        with np.errstate(over="ignore", invalid="ignore"):
            # beyond the FP32 range a_up is inf, tau is inf and the check fails closed
            self.a_up = round_up_f32(sum_up(np.abs(self.W_blocks).sum(axis=1), block))


class BlockedChecker:
    """One random-sign checksum per block of ``block`` rows (reference
    `src/pck/checker.py:27-99`):

        rho = (r^T W_beta) . x - r . y_beta
        tau = (gamma_h + u32) (a_beta . |x|) + eps,  every part rounded up,

    and a block passes only if its outputs are finite, tau is finite and |rho| <= tau.
    """

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
        self.m, self.n = m, n
        self.block = block
        self.num_blocks = m // block
        self.W_blocks = bank.W_blocks
        self.x = x.astype(np.float64)
        with np.errstate(over="ignore", invalid="ignore"):
            self.abs_bound: NDArray[np.float64] = sum_up(bank.a_up @ np.abs(self.x), n)
        self.gamma_h = gamma(height)
        self.coef = next_up(next_up(self.gamma_h) + U32)

    @property
    def tau_base(self) -> NDArray[np.float64]:
        """(gamma_h + u32) (a_beta . |x|) per block, rounded up (reference
        `src/pck/checker.py:68-73`)."""
        with np.errstate(over="ignore", invalid="ignore"):
            return np.nextafter(self.coef * self.abs_bound, np.inf)

    def verdict_with_signs(
        self, y: NDArray[np.floating], signs: NDArray[np.floating]
    ) -> tuple[NDArray[np.bool_], NDArray[np.float64], NDArray[np.float64]]:
        """(passed, rho, tau), each (K, nb), for explicit signs of shape (K, nb, block).

        One check of `src/pck/checker.py:89-98` per sign draw k.
        """
        if y.shape != (self.m,):
            raise ValueError(f"y has shape {y.shape}, expected ({self.m},)")
        r_all = np.asarray(signs, dtype=np.float64).reshape(-1, self.num_blocks, self.block)
        with np.errstate(invalid="ignore", over="ignore"):
            yb = y.astype(np.float64).reshape(self.num_blocks, self.block)
        finite = np.isfinite(yb).all(axis=1)
        passed, rhos, taus = [], [], []
        for r in r_all:
            c = np.einsum("kb,kbn->kn", r, self.W_blocks).astype(np.float32).astype(np.float64)
            with np.errstate(invalid="ignore", over="ignore"):
                rho = c @ self.x - (r * yb).sum(axis=1)
                mags = sum_up(np.abs(c) @ np.abs(self.x), self.n) + sum_up(
                    np.abs(yb).sum(axis=1), self.block
                )
                eps = np.nextafter(next_up(gamma(self.n + self.block + 1, U64)) * mags, np.inf)
                tau = np.nextafter(self.tau_base + eps, np.inf)
                ok = finite & np.isfinite(tau) & (np.abs(rho) <= tau)
            passed.append(ok)
            rhos.append(rho)
            taus.append(tau)
        return np.array(passed), np.array(rhos), np.array(taus)

    def verdict(
        self, y: NDArray[np.floating], rng: np.random.Generator, checks: int = 1
    ) -> NDArray[np.bool_]:
        """Per-block verdict after ``checks`` sign draws from ``rng`` (reference
        `src/pck/checker.py:75-99`, same draw order: one (nb, block) draw per check)."""
        if y.shape != (self.m,):
            raise ValueError(f"y has shape {y.shape}, expected ({self.m},)")
        ok = np.ones(self.num_blocks, dtype=bool)
        for _ in range(checks):
            r = rng.choice([-1.0, 1.0], (self.num_blocks, self.block))
            ok &= self.verdict_with_signs(y, r[None])[0][0]
        return ok


def gpu_threshold_exact(
    a: NDArray[np.floating],
    x: NDArray[np.floating],
    y: NDArray[np.floating],
    block: int,
    coef: float,
    geps: float,
    tau_floor: float,
) -> list[Fraction]:
    """Exact tau per block of the GPU formula from the stored bank (reference
    `src/pck/cuda/csrc/checker_kernel.cu:176-181`):

        s   = a_beta . |x|
        tau = coef s + geps ((1 + u32) s + sum_{i in beta} |y_i|) + tau_floor

    in rational arithmetic (no rounding at all).  ``a`` is the stored BF16 bank (nb, n) as
    floats, ``x`` the BF16 activations, ``y`` the FP32 outputs.
    """
    nb = a.shape[0]
    xs = [abs(Fraction(float(v))) for v in x]
    yb = np.asarray(y, dtype=np.float64).reshape(nb, block)
    one_u = 1 + Fraction(U32)
    out = []
    for beta in range(nb):
        s = sum((Fraction(float(aj)) * xj for aj, xj in zip(a[beta], xs) if aj), Fraction(0))
        ysum = sum((abs(Fraction(float(v))) for v in yb[beta]), Fraction(0))
        out.append(
            Fraction(coef) * s + Fraction(geps) * (one_u * s + ysum) + Fraction(tau_floor)
        )
    return out


def gpu_rho_exact(
    c: NDArray[np.floating], r: NDArray[np.integer], x: NDArray[np.floating], y: NDArray[np.floating]
) -> NDArray[np.float64]:
    """rho = c . x - r . y_beta per (check, block), exactly, rounded once to FP64.

    ``c`` (K, nb, n) and ``r`` (K, nb, b) are the stored bank; ``x`` and ``y`` as in
    `gpu_threshold_exact`.  Used to bound the HIP checker's own rounding of rho.
    """
    K, nb, _ = c.shape
    b = r.shape[2]
    xs = [Fraction(float(v)) for v in x]
    yb = np.asarray(y, dtype=np.float64).reshape(nb, b)
    out = np.empty((K, nb))
    for k in range(K):
        for beta in range(nb):
            cx = sum((Fraction(float(cj)) * xj for cj, xj in zip(c[k, beta], xs) if cj), Fraction(0))
            ry = sum(
                (Fraction(float(yi)) * int(ri) for ri, yi in zip(r[k, beta], yb[beta])), Fraction(0)
            )
            out[k, beta] = float(cx - ry)
    return out
