"""TEST INFRASTRUCTURE — CPU model of the in-pass checksums and the row-sum check.

The in-pass GEMV writes, beside y = W x, one pair per output row from the FP32 products
p_j = fl32(W_ij x_j) the tree forms anyway (exact barring FP32 underflow):

    d_i = sum over consecutive pairs (p_2k + p_2k+1), each pair added in FP32, the pair sums
          widened and added in FP64 (round to nearest);
    s_i = sum_j |p_j| in FP32 (round to nearest), stored widened to FP64.

The row-sum check then decides every (check, block) pair of the blocked checker (reference
relation `src/pck/cuda/csrc/checker_kernel.cu:115-183`, bank quantities replaced):

    rho = sum_i r_i d_i - sum_i r_i y_i
    s   = up_to_f32(RU(s_factor * RU(sum_i s_i)))
    tau = coef s + geps ((1 + u32) s + RU(sum_i |y_i|)) + tau_floor   (every operation upward)
    passed = every y_i finite and tau finite and |rho| <= tau.

`row_sums` and `rowsum_check_with_signs` reproduce the GPU's bits: the same summation order
(lane l of a row's L = min(T, 64) lanes takes vector positions, then chains, then the columns
of each vector in order; an xor butterfly across lanes; the check's lane l adds rows l, l + 64,
... and an xor butterfly) and the same directed-rounding steps (error-free transformations plus
a one-ulp raise, as the library's device code forms them).  `exact_rowsum_threshold` is the
threshold for the exact S = sum |W_ij x_j| in rational arithmetic, against which the rounded
one is pinned.
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
from numpy.typing import NDArray

from pck.fp import U32, U64, gamma, next_up

WAVE = 64


def depth_of(n: int, threads: int, vec: int) -> int:
    """The most additions a product passes through in `row_sums` for one launch shape: a lane's
    sequential terms, then the butterfly levels."""
    lanes = min(threads, WAVE)
    positions = -(-(-(-n // vec)) // threads)
    return (threads // lanes) * positions * vec + int(math.log2(lanes))


def rowsum_constants(n: int, block: int, height: int) -> dict[str, float]:
    """coef, geps, tau_floor and s_factor of a row-sum check (the host's formulas).  coef is
    the bank checker's gamma_h + u32 (reference `src/pck/cuda/checker.py:106-125`): its u32 term
    covered c's FP32 rounding there and covers the FP32 pair sums of d here (at most
    u32 sum |p| per row).  With D the largest `depth_of` over thread counts 32..1024 and
    vectors of 8 and 16: s_factor = 1 + (D + 1) 2^-23 >= 1 / (1 - gamma_D(u32)) bounds the FP32
    sums of |p|; geps = gamma_H(u64), H = D + ceil(b / 64) + 7, bounds rho's FP64 evaluation;
    tau_floor = n 2^-148 + 2 b n 2^-150 adds what FP32 product underflow may take from d and
    s (at most 2^-150 per product)."""
    D = max(depth_of(n, t, v) for t in (32, 64, 128, 256, 512, 1024) for v in (8, 16))
    return {
        "coef": next_up(gamma(height) + U32, 2),
        "geps": next_up(gamma(D + -(-block // WAVE) + 7, U64), 2),
        "tau_floor": next_up(n * 2.0**-148 + 2 * block * n * 2.0**-150, 2),
        "s_factor": next_up(1.0 + (D + 1) * 2.0**-23, 2),
    }


def row_sums(
    W: NDArray[np.floating], x: NDArray[np.floating], threads: int = 256, vec: int = 8,
    chunk_rows: int = 2048,
) -> NDArray[np.float64]:  # fmt: skip
    """(m, 2) FP64 (d_i, s_i) with the GPU's bits.

    ``W`` holds the weight values (BF16 or decoded E4M3) and ``x`` the BF16 activations, as
    floats; ``vec`` is 8 for BF16 weights and 16 for E4M3.  Lane l of L = min(threads, 64)
    owns the chains t = l + L j (j < C = threads / L) of the coalesced tree, each with its own
    d (FP64) and s (FP32), from +0; for each vector position v, for each chain j, it takes the
    ``vec`` products of vector v threads + t (FP32, columns past n as +0) and adds, pair by pair,
    fl32(p_k + p_k+1) to d_j and |p_k| then |p_k+1| to s_j.  The chains combine in halving
    order (for half = C/2, ..., 1: chain i += chain i + half), then for off = L/2, ..., 1 every
    lane adds its partner's d and s (lane ^ off), in FP64 and FP32.
    """
    m, n = W.shape
    lanes = min(threads, WAVE)
    chains = threads // lanes
    per_lane = -(-(-(-n // vec)) // threads)
    width = per_lane * threads * vec
    lane_idx = np.arange(lanes)
    xs = np.zeros(width, dtype=np.float32)
    xs[:n] = np.asarray(x, dtype=np.float32)
    out = np.empty((m, 2))
    with np.errstate(under="ignore", over="ignore", invalid="ignore"):
        for r0 in range(0, m, chunk_rows):
            Wc = np.zeros((min(chunk_rows, m - r0), width), dtype=np.float32)
            Wc[:, :n] = W[r0 : r0 + chunk_rows]
            p = Wc * xs  # FP32 products, as the tree forms them
            d = np.zeros((chains, p.shape[0], lanes))
            s = np.zeros((chains, p.shape[0], lanes), dtype=np.float32)
            for v in range(per_lane):
                for j in range(chains):
                    base = (v * threads + lanes * j + lane_idx) * vec
                    for k in range(0, vec, 2):
                        p0, p1 = p[:, base + k], p[:, base + k + 1]
                        d[j] = d[j] + (p0 + p1).astype(np.float64)
                        s[j] = s[j] + np.abs(p0)
                        s[j] = s[j] + np.abs(p1)
            half = chains // 2
            while half > 0:  # chain i += chain i + half
                d[:half] = d[:half] + d[half : 2 * half]
                s[:half] = s[:half] + s[half : 2 * half]
                half //= 2
            d, s = d[0], s[0]
            off = lanes // 2
            while off > 0:
                d = d + d[:, lane_idx ^ off]
                s = s + s[:, lane_idx ^ off]
                off //= 2
            out[r0 : r0 + p.shape[0], 0] = d[:, 0]
            out[r0 : r0 + p.shape[0], 1] = s[:, 0].astype(np.float64)
    return out


# --- directed rounding, step for step as the device code forms it ----------------------------

DBL_MAX = np.finfo(np.float64).max


def _raise_bits(v: float) -> float:
    """The float whose bit pattern is v's plus one (the device's one-ulp raise of v >= 0)."""
    return float(np.array([np.array([v]).view(np.int64)[0] + 1], dtype=np.int64).view(np.float64)[0])


def next_up_dev(v: float) -> float:
    """The device's next_up: NaN and +inf unchanged, +-0 to the smallest subnormal."""
    if math.isnan(v) or v == math.inf:
        return v
    if v == 0.0:
        return 5e-324
    return math.nextafter(v, math.inf)


def add_up_nonneg(a: float, b: float) -> float:
    """RU(a + b) for a, b >= 0: the RN sum raised by one ulp when its exact error is positive;
    +inf stays +inf."""
    s = a + b
    if math.isinf(s) or math.isnan(s):
        return s
    return _raise_bits(s) if Fraction(a) + Fraction(b) > Fraction(s) else s


def mul_up_nonneg(a: float, b: float) -> float:
    """RU(a b) for a, b >= 0: raised by one ulp when the exact residual is positive or the
    product lies below 2^-960 (where the device's FMA residual may be inexact)."""
    p = a * b
    if math.isnan(p) or math.isinf(p):
        return p
    if p < 2.0**-960:
        return _raise_bits(p)
    return _raise_bits(p) if Fraction(a) * Fraction(b) > Fraction(p) else p


def add_up(a: float, b: float) -> float:
    s = a + b
    if s == -math.inf and a != -math.inf and b != -math.inf:
        return -DBL_MAX
    if math.isnan(s) or math.isinf(s):
        return s
    return next_up_dev(s) if Fraction(a) + Fraction(b) > Fraction(s) else s


def mul_up(a: float, b: float) -> float:
    p = a * b
    if math.isnan(p) or p == math.inf:
        return p
    if p == -math.inf:
        return p if (math.isinf(a) or math.isinf(b)) else -DBL_MAX
    if p == 0.0:
        return p if (a == 0.0 or b == 0.0) else next_up_dev(p)
    if abs(p) < 2.0**-960:
        return next_up_dev(p)
    return next_up_dev(p) if Fraction(a) * Fraction(b) > Fraction(p) else p


def up_to_f32(v: float) -> float:
    """The smallest FP32 value >= v (v >= 0), as a float; +inf beyond the FP32 range."""
    with np.errstate(over="ignore"):
        f = np.float32(v)
    if float(f) < v:
        f = np.array([np.array([f]).view(np.uint32)[0] + 1], dtype=np.uint32).view(np.float32)[0]
    return float(f)


def _add_up_nonneg_vec(a: NDArray[np.float64], b: NDArray[np.float64]) -> NDArray[np.float64]:
    """Elementwise add_up_nonneg with the device's TwoSum (exact in FP64 barring overflow)."""
    with np.errstate(invalid="ignore", over="ignore"):
        s = a + b
        bv = s - a
        err = (a - (s - bv)) + (b - bv)
        raised = (s.view(np.int64) + 1).view(np.float64)
        return np.where(err > 0, raised, s)


def rowsum_check_with_signs(
    sums: NDArray[np.float64], y: NDArray[np.floating], signs: NDArray[np.integer],
    block: int, coef: float, geps: float, tau_floor: float, s_factor: float,
) -> tuple[NDArray[np.bool_], NDArray[np.float64], NDArray[np.float64]]:  # fmt: skip
    """(passed, rho, tau), each (K, nb), with the GPU's bits for signs (K, nb, block)."""
    r_all = np.asarray(signs).reshape(-1, sums.shape[0] // block, block)
    K, nb, _ = r_all.shape
    lanes = np.arange(WAVE)
    passed = np.zeros((K, nb), dtype=bool)
    rhos = np.zeros((K, nb))
    taus = np.zeros((K, nb))
    d_all = sums[:, 0].reshape(nb, block)
    s_all = sums[:, 1].reshape(nb, block)
    y_all = np.asarray(y, dtype=np.float32).astype(np.float64).reshape(nb, block)
    for k in range(K):
        for beta in range(nb):
            cx = np.zeros(WAVE)
            ry = np.zeros(WAVE)
            s = np.zeros(WAVE)
            ya = np.zeros(WAVE)
            neg = r_all[k, beta] < 0
            with np.errstate(invalid="ignore", over="ignore"):
                for i0 in range(0, block, WAVE):
                    rows = np.arange(i0, min(i0 + WAVE, block))
                    ln = rows - i0
                    dv = np.where(neg[rows], -d_all[beta, rows], d_all[beta, rows])
                    yv = np.where(neg[rows], -y_all[beta, rows], y_all[beta, rows])
                    cx[ln] = cx[ln] + dv
                    ry[ln] = ry[ln] + yv
                    s[ln] = _add_up_nonneg_vec(s[ln], s_all[beta, rows])
                    ya[ln] = _add_up_nonneg_vec(ya[ln], np.abs(y_all[beta, rows]))
                off = WAVE // 2
                while off > 0:
                    cx = cx + cx[lanes ^ off]
                    ry = ry + ry[lanes ^ off]
                    s = _add_up_nonneg_vec(s, s[lanes ^ off])
                    ya = _add_up_nonneg_vec(ya, ya[lanes ^ off])
                    off //= 2
            s_up = up_to_f32(mul_up_nonneg(float(s[0]), s_factor))
            rho = float(cx[0]) - float(ry[0])
            cabs_up = mul_up(1.0 + U32, s_up)
            eps = mul_up(geps, add_up(cabs_up, float(ya[0])))
            tau = add_up(add_up(mul_up(coef, s_up), eps), tau_floor)
            passed[k, beta] = math.isfinite(ya[0]) and math.isfinite(tau) and abs(rho) <= tau
            rhos[k, beta] = rho
            taus[k, beta] = tau
    return passed, rhos, taus


def exact_rowsum_threshold(
    W: NDArray[np.floating], x: NDArray[np.floating], y: NDArray[np.floating], block: int,
    coef: float, geps: float, tau_floor: float,
) -> list[Fraction]:  # fmt: skip
    """tau per block with exact S = sum_{i in beta} sum_j |W_ij x_j| and exact sum |y|, in
    rational arithmetic (no rounding): the value the rounded threshold must never fall below."""
    m, n = W.shape
    xs = [abs(Fraction(float(v))) for v in x]
    one_u = 1 + Fraction(U32)
    out = []
    for beta in range(m // block):
        S = Fraction(0)
        for i in range(beta * block, (beta + 1) * block):
            S += sum((abs(Fraction(float(w))) * xj for w, xj in zip(W[i], xs) if w), Fraction(0))
        Y = sum((abs(Fraction(float(v))) for v in y[beta * block : (beta + 1) * block]), Fraction(0))
        out.append(Fraction(coef) * S + Fraction(geps) * (one_u * S + Y) + Fraction(tau_floor))
    return out


def exact_rho(
    W: NDArray[np.floating], x: NDArray[np.floating], y: NDArray[np.floating],
    signs: NDArray[np.integer], block: int,
) -> list[list[Fraction]]:  # fmt: skip
    """r^T (W x) - r^T y per (check, block), exactly."""
    m, n = W.shape
    xs = [Fraction(float(v)) for v in x]
    dx = [sum((Fraction(float(w)) * xj for w, xj in zip(W[i], xs) if w), Fraction(0)) for i in range(m)]
    r_all = np.asarray(signs).reshape(-1, m // block, block)
    return [
        [
            sum(
                (int(r_all[k, beta, i]) * (dx[beta * block + i] - Fraction(float(y[beta * block + i])))
                 for i in range(block)),
                Fraction(0),
            )
            for beta in range(m // block)
        ]
        for k in range(r_all.shape[0])
    ]
