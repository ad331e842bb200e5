"""TEST INFRASTRUCTURE — bit-level CPU models of two GPU blocked checkers' arithmetic.

Both evaluate, per (check k, block beta), the reference relation

    rho = c . x - r . y_beta
    s   = a . |x|                       rounded upward
    tau = coef s + geps ((1 + u32) s + sum |y_beta|) + tau_floor,  every operation upward
    passed = every y finite, tau finite, |rho| <= tau

and differ only in how they round on the way.

`reference_gpu_check` restates the reference's CUDA kernel
(`src/pck/cuda/csrc/checker_kernel.cu:63-183`) operation by operation:

- the n columns are split into `segments` pieces of seg_len = ceil(n / segments) columns
  (`bindings.cpp:209`);
- thread t of 256 takes columns seg * seg_len + t, + 256, ... of its segment, and keeps:
  - c . x as a Dot2 chain in FP32: TwoProduct by FMA, TwoSum, error terms in lo
    (`checker_kernel.cu:115-127`), then hi + lo in FP64;
  - s = RU32(s + RU32(a_j |x_j|)) in FP32 (`:128`);
- the block sums (`block_sum`, `:63-85`) halve within each 32-lane warp (lane i += lane
  i + off, off = 16 .. 1), then halve the eight warp sums, zero-padded to 32 lanes, in FP64
  (c . x to nearest, s upward);
- the segments' partials are added in segment order from 0 (`:169-173`);
- r . y in FP64 to nearest, and sum |y| in FP32 upward, per thread over rows t, t + 256, ...,
  are block-summed the same way;
- tau's products and sums are rounded upward in FP64 (`:176-181`).

`hip_check` restates this build's kernel (`proof-carrying-kernels_amd/csrc/check_pair.h`):

- lane t of 256 takes the y rows t, t + 256, ...: r . y to nearest, sum |y| upward, in FP64;
- it then takes the bank quads t, t + 256, ... (n % 4 == 0), column i of each quad into
  accumulator i:
  - c . x by FMA in FP64 (the product c_j x_j is exact in FP64, so one rounding, the add's);
  - a_j |x_j| exact in FP64, added upward;
- the remaining columns j (all of them when n % 4 != 0) go into accumulator j % 4;
- the four accumulators combine as (0 + 2) + (1 + 3);
- the lanes combine by a 64-lane butterfly over lane distances 1, 2, 4, ..., 32, which gives
  lane 0 the adjacent-pair tree ((v0 + v1) + (v2 + v3)) + ..., and the four waves as
  (0 + 2) + (1 + 3);
- s stays in FP64 (+inf beyond the FP32 range), and tau is formed with `rounding.h`'s mul_up
  and add_up, including mul_up's one-ulp raise of a nonzero product below 2^-960.

Directed roundings are computed exactly:
- in FP32 from the exact FP64 value, which a TwoSum error corrects when the FP64 sum itself
  rounded;
- in FP64 through `fractions.Fraction`.

Pinned by (`tests/test_oracle_checker_orders.py`):
- small-integer inputs, on which every operation is exact, so both models give the exact
  rational threshold and rho;
- the reference test's own criterion (`tests/gpu/test_checker_cuda.py:54-80`): tau at or above
  the exact threshold and at most about n 2^-24 above it;
- rho within the threshold's own rounding allowance of the exact value;
- a hand-traced case in which the FP32 upward chain and the FP64 sum differ.

The GPU test `tests/gpu/test_checker_gpu.py` compares the HIP kernel's passed, rho and tau
with `hip_check` bit for bit.
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
from numpy.typing import NDArray

THREADS = 256
WARP = 32
WAVE = 64
ONE_PLUS_U32 = 1.0 + 2.0**-24

F64 = NDArray[np.float64]


def _two_sum_err(a: F64, b: F64, s: F64) -> F64:
    """Exact error (a + b) - s of s = RN(a + b) (Knuth's TwoSum), for finite s."""
    with np.errstate(invalid="ignore", over="ignore"):
        bv = s - a
        return (a - (s - bv)) + (b - bv)


def add_up64(a: F64, b: F64) -> F64:
    """RU(a + b) in FP64 for finite or +inf operands whose sum is not -inf."""
    with np.errstate(invalid="ignore", over="ignore"):
        s = a + b
        err = _two_sum_err(a, b, s)
        return np.where(np.isfinite(s) & (err > 0), np.nextafter(s, np.inf), s)


def up_to_f32(v: F64) -> F64:
    """The smallest FP32 value >= v, widened to FP64 (+inf past the FP32 range)."""
    with np.errstate(over="ignore", invalid="ignore"):
        f = np.asarray(v, dtype=np.float64).astype(np.float32)
        f = np.where(f.astype(np.float64) < v, np.nextafter(f, np.float32(np.inf)), f)
    return f.astype(np.float64)


def add_up32(a: F64, b: F64) -> F64:
    """RU32(a + b) for FP32 values a, b (held in FP64)."""
    with np.errstate(invalid="ignore", over="ignore"):
        s = a + b
        err = _two_sum_err(a, b, s)
        f = up_to_f32(s)
        on_grid = f == s
        return np.where(on_grid & (err > 0) & np.isfinite(s),
                        np.nextafter(f.astype(np.float32), np.float32(np.inf)).astype(np.float64), f)  # fmt: skip


def _ru(q: Fraction) -> float:
    """The smallest double >= q (q finite and within the double range)."""
    f = float(q)
    if Fraction(f) < q:
        f = math.nextafter(f, math.inf)
    return f


def _ru_mul(a: float, b: float) -> float:
    if not (math.isfinite(a) and math.isfinite(b)):
        return a * b
    return _ru(Fraction(a) * Fraction(b))


def _ru_add(a: float, b: float) -> float:
    if not (math.isfinite(a) and math.isfinite(b)):
        return a + b
    return _ru(Fraction(a) + Fraction(b))


def _halve(v: F64, width: int, up: bool) -> F64:
    """Halving sum over the last axis (length ``width``, a power of two): a[i] += a[i + off]
    for off = width / 2, ..., 1; the result of lane 0."""
    v = v.copy()
    off = width // 2
    while off:
        lo, hi = v[..., :off], v[..., off : 2 * off]
        v[..., :off] = add_up64(lo, hi) if up else lo + hi
        off //= 2
    return v[..., 0]


def _pairs_up(v: F64, up: bool) -> F64:
    """Adjacent-pair tree over the last axis (a power of two): ((v0 + v1) + (v2 + v3)) + ...,
    lane 0's result of a butterfly over distances 1, 2, 4, ..."""
    while v.shape[-1] > 1:
        v = add_up64(v[..., 0::2], v[..., 1::2]) if up else v[..., 0::2] + v[..., 1::2]
    return v[..., 0]


def _block_sum(v: F64, up: bool) -> F64:
    """The reference's `block_sum` over (..., 256) thread values: each warp of 32 halves, then
    lanes 0-7 of warp 0 hold the eight warp sums and lanes 8-31 zero, halved again."""
    warps = _halve(v.reshape(*v.shape[:-1], THREADS // WARP, WARP), WARP, up)
    padded = np.zeros((*v.shape[:-1], WARP))
    padded[..., : THREADS // WARP] = warps
    return _halve(padded, WARP, up)


def _y_terms(r: NDArray, y: F64, up32: bool) -> tuple[F64, F64, NDArray[np.bool_]]:
    """Per (pair, lane): r . y to nearest in FP64 and sum |y| upward (in FP32 with ``up32``,
    else in FP64) over rows lane, lane + 256, ...; and whether the block has a non-finite y.
    ``r`` (P, b) signs, ``y`` (P, b) the block's outputs for each pair."""
    P, b = y.shape
    ry = np.zeros((P, THREADS))
    ya = np.zeros((P, THREADS))
    for i0 in range(0, b, THREADS):
        cnt = min(THREADS, b - i0)
        yi = y[:, i0 : i0 + cnt]
        with np.errstate(invalid="ignore"):
            ry[:, :cnt] = ry[:, :cnt] + np.where(r[:, i0 : i0 + cnt] > 0, yi, -yi)
        ya[:, :cnt] = (add_up32 if up32 else add_up64)(ya[:, :cnt], np.abs(yi))
    return ry, ya, ~np.isfinite(y).all(axis=1)


def reference_default_segments(n: int, checks: int, num_blocks: int, sms: int) -> int:
    """The reference's default segment count (`src/pck/cuda/checker.py:108-111`): about four
    CUDA blocks per SM, each segment at least 512 columns (30 SMs on its RTX 5060)."""
    wanted = -(-4 * sms // (checks * num_blocks))
    return max(1, min(wanted, n // 512))


def _pairs(c: NDArray, r: NDArray, y: NDArray) -> tuple[F64, NDArray, F64, NDArray, int]:
    """Flattens (K, nb, n) c and (K, nb, b) r to pairs p = k nb + beta, with each pair's y block
    and its block index."""
    K, nb, n = c.shape
    b = r.shape[2]
    yb = np.asarray(y, dtype=np.float32).astype(np.float64).reshape(nb, b)
    beta = np.tile(np.arange(nb), K)
    return (np.asarray(c, np.float32).astype(np.float64).reshape(K * nb, n),
            np.asarray(r).reshape(K * nb, b), yb[beta], beta, n)  # fmt: skip


def _finish(cx: F64, ry: F64, s: F64, yabs: F64, bad: NDArray[np.bool_], coef: float,
            geps: float, tau_floor: float, mul_up, add_up, K: int, nb: int):  # type: ignore[no-untyped-def]  # fmt: skip
    rho = cx - ry
    tau = np.empty_like(rho)
    for p in range(rho.size):
        sp, ya = float(s[p]), float(yabs[p])
        cabs = mul_up(ONE_PLUS_U32, sp)
        eps = mul_up(geps, add_up(cabs, ya))
        tau[p] = add_up(add_up(mul_up(coef, sp), eps), tau_floor)
    with np.errstate(invalid="ignore"):
        passed = ~bad & np.isfinite(tau) & (np.abs(rho) <= tau)
    return passed.reshape(K, nb), rho.reshape(K, nb), tau.reshape(K, nb)


def reference_gpu_check(c, a, r, x, y, coef: float, geps: float, tau_floor: float,  # type: ignore[no-untyped-def]
                        segments: int) -> tuple[NDArray[np.bool_], F64, F64]:  # fmt: skip
    """(passed, rho, tau), each (K, nb), with the bits of the reference's CUDA kernel.

    ``c`` (K, nb, n) FP32 checksums, ``a`` (nb, n) BF16 column sums (as floats), ``r`` (K, nb, b)
    signs, ``x`` (n,) BF16 activations, ``y`` (m,) FP32 outputs (as floats)."""
    c2, r2, yb, beta, n = _pairs(c, r, y)
    K, nb = c.shape[0], c.shape[1]
    a2 = np.asarray(a, np.float32).astype(np.float64)[beta]
    x64 = np.asarray(x, np.float32).astype(np.float64)
    P = c2.shape[0]
    seg_len = -(-n // segments)
    cx_total = np.zeros(P)
    s_total = np.zeros(P)
    for seg in range(segments):
        lo_col, hi_col = seg * seg_len, min(n, (seg + 1) * seg_len)
        hi = np.zeros((P, THREADS), np.float32)
        lo = np.zeros((P, THREADS), np.float32)
        s = np.zeros((P, THREADS))
        for j0 in range(lo_col, hi_col, THREADS):
            cnt = min(THREADS, hi_col - j0)
            cj = c2[:, j0 : j0 + cnt].astype(np.float32)
            xj = x64[j0 : j0 + cnt].astype(np.float32)
            exact = cj.astype(np.float64) * xj.astype(np.float64)  # exact in FP64
            p = exact.astype(np.float32)
            e = (exact - p.astype(np.float64)).astype(np.float32)  # fma(c, x, -p)
            h = hi[:, :cnt]
            total = h + p
            z = total - h
            err = (h - (total - z)) + (p - z)
            hi[:, :cnt] = total
            lo[:, :cnt] = lo[:, :cnt] + (err + e)
            term = up_to_f32(a2[:, j0 : j0 + cnt] * np.abs(x64[j0 : j0 + cnt]))
            s[:, :cnt] = add_up32(s[:, :cnt], term)
        cx = hi.astype(np.float64) + lo.astype(np.float64)
        cx_total = cx_total + _block_sum(cx, up=False)
        s_total = add_up64(s_total, _block_sum(s, up=True))
    ry, ya, bad = _y_terms(r2, yb, up32=True)
    ry_total = _block_sum(ry, up=False)
    ya_total = _block_sum(ya, up=True)
    return _finish(cx_total, ry_total, s_total, ya_total, bad, coef, geps, tau_floor,
                   _ru_mul, _ru_add, K, nb)  # fmt: skip


def _hip_mul_up(a: float, b: float) -> float:
    """`rounding.h` mul_up: exact RU(a b), except that a nonzero product below 2^-960 in
    magnitude is raised one ulp from its round-to-nearest value."""
    p = a * b
    if not math.isfinite(p) or (p == 0.0 and (a == 0.0 or b == 0.0)):
        return p
    if p == 0.0 or abs(p) < 2.0**-960:
        return math.nextafter(p, math.inf)
    return _ru(Fraction(a) * Fraction(b))


def hip_check(c, a, r, x, y, coef: float, geps: float, tau_floor: float  # type: ignore[no-untyped-def]
              ) -> tuple[NDArray[np.bool_], F64, F64]:  # fmt: skip
    """(passed, rho, tau), each (K, nb), with the bits of this build's HIP checker
    (`check_pair.h`); arguments as for `reference_gpu_check`."""
    c2, r2, yb, beta, n = _pairs(c, r, y)
    K, nb = c.shape[0], c.shape[1]
    a2 = np.asarray(a, np.float32).astype(np.float64)[beta]
    x64 = np.asarray(x, np.float32).astype(np.float64)
    P = c2.shape[0]
    ry, ya, bad = _y_terms(r2, yb, up32=False)
    cx = np.zeros((4, P, THREADS))
    sa = np.zeros((4, P, THREADS))
    lanes = np.arange(THREADS)
    nq = n // 4 if n % 4 == 0 else 0
    for q0 in range(0, nq, THREADS):  # quad q0 + lane, columns 4q .. 4q + 3 -> accumulators
        cnt = min(THREADS, nq - q0)
        for i in range(4):
            cols = 4 * (q0 + lanes[:cnt]) + i
            prod = c2[:, cols] * x64[cols]
            cx[i, :, :cnt] = prod + cx[i, :, :cnt]
            sa[i, :, :cnt] = add_up64(sa[i, :, :cnt], a2[:, cols] * np.abs(x64[cols]))
    if nq == 0:  # element columns j = lane, lane + 256, ...: all in accumulator lane % 4
        e_cx = np.zeros((P, THREADS))
        e_sa = np.zeros((P, THREADS))
        for j0 in range(0, n, THREADS):
            cnt = min(THREADS, n - j0)
            cols = j0 + lanes[:cnt]
            e_cx[:, :cnt] = c2[:, cols] * x64[cols] + e_cx[:, :cnt]
            e_sa[:, :cnt] = add_up64(e_sa[:, :cnt], a2[:, cols] * np.abs(x64[cols]))
        for i in range(4):
            mine = lanes % 4 == i
            cx[i][:, mine] = e_cx[:, mine]
            sa[i][:, mine] = e_sa[:, mine]
    q_cx = (cx[0] + cx[2]) + (cx[1] + cx[3])
    q_s = add_up64(add_up64(sa[0], sa[2]), add_up64(sa[1], sa[3]))

    def group(v: F64, up: bool) -> F64:
        waves = _pairs_up(v.reshape(P, THREADS // WAVE, WAVE), up)  # (P, 4)
        add = add_up64 if up else (lambda u, w: u + w)
        return add(add(waves[:, 0], waves[:, 2]), add(waves[:, 1], waves[:, 3]))

    cx_t, s_t, ry_t, ya_t = group(q_cx, False), group(q_s, True), group(ry, False), group(ya, True)
    s_up = np.where(s_t <= float(np.finfo(np.float32).max), s_t, np.inf)
    bad = bad | ~np.isfinite(ya_t)
    return _finish(cx_t, ry_t, s_up, ya_t, bad, coef, geps, tau_floor, _hip_mul_up, _ru_add, K, nb)
