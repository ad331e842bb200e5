"""Measures, on the GPU, the device arithmetic that the error bounds assume (probes of
libpck_probe.so, built with the library's flags), against exact host arithmetic.

- ``expf``: the membership and sampling bounds assume a device expf within 2 ulp (reference
  `src/pck/member.py:84-102`).  Every FP32 x in [-128, -2^-26] (276,824,065 values) is checked
  against the FP64 exponential, and a sample of (-2^-26, 0]; the error must be at most 2 ulp
  of the exact value's FP32 spacing (measured: below 1 ulp).
- ``v_mfma_f64_16x16x4_f64``: the batched checker's c . x assumes every operation rounds to
  nearest.  Measured: each output is four IEEE FMAs in K order, each rounded once to nearest
  even, continued across chained steps.  Crafted cases separate this from one rounding of the
  exact sum, from rounded products, from a pairwise tree and from truncation; random full
  53-bit operands (where a rounded product differs from an FMA) and the checker's own operand
  kind (FP32 x BF16) follow it exactly.
- ``v_mfma_f32_32x32x16_bf16`` with one populated group of 8 K-slots and a zero accumulator
  (the batched product's step): every output equals `oracle.batched.mfma_step`, with either
  lane half populated, for crafted and random operands.
- ``v_mfma_f32_16x16x32_bf16`` on non-negative operands (the batched checker's a . |x|): a
  step never falls below the exact sum by more than 2^-18 + 2^-24 relative (plus 33 x 2^-126),
  which the checker's round-up factor 1 + 2^-16 covers.
- ``rounding.h``: on non-negative operands the branch-free mul_up_pos and add_up_nonneg give
  the general mul_up and add_up bits (zeros, subnormals, products underflowing to 0 or below
  2^-960, overflow, inf, NaN), and mul_up is the exact upward product except one ulp above it
  for nonzero products below 2^-960.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle.batched import mfma_step
from pck.cuda import probe
from tests.golden.make_mfma_step_fixture import crafted

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def ulp_errors(x: np.ndarray) -> np.ndarray:
    """|expf(x) - e^x| in units of the FP32 spacing at e^x (2^-149 at least)."""
    y = probe.expf(torch.from_numpy(x).cuda()).cpu().numpy().astype(np.float64)
    e = np.exp(x.astype(np.float64))
    spacing = np.maximum(np.spacing(e.astype(np.float32)).astype(np.float64), 2.0**-149)
    return np.abs(y - e) / spacing


def test_expf_within_two_ulp_on_every_float_in_minus_128_to_0() -> None:
    lo = int(np.float32(2.0**-26).view(np.uint32))
    hi = int(np.float32(128.0).view(np.uint32))
    worst, count = 0.0, 0
    for start in range(lo, hi + 1, 1 << 24):
        bits = np.arange(start, min(start + (1 << 24), hi + 1), dtype=np.uint32) | np.uint32(1 << 31)
        err = ulp_errors(bits.view(np.float32))
        worst, count = max(worst, float(err.max())), count + err.size
    print(f"expf over [-128, -2^-26]: {count} values, max error {worst:.6f} ulp", flush=True)
    assert count == hi - lo + 1
    assert worst <= 2.0
    tiny = -np.random.default_rng(0).uniform(0, 2.0**-26, 1 << 20).astype(np.float32)
    assert float(ulp_errors(np.append(tiny, np.float32(-0.0))).max()) <= 2.0


# ---- FP64 matrix core ---------------------------------------------------------------------


def fma(a: float, b: float, c: float) -> float:
    return float(Fraction(a) * Fraction(b) + Fraction(c))  # one rounding, to nearest even


def fma_chain(a: list[float], b: list[float], c: float) -> float:
    for x, y in zip(a, b, strict=True):
        c = fma(x, y, c)
    return c


E = 2.0**-52
CASES = [  # (a[0..3], b[0..3], c), each with a note of what it separates
    ([1.0, 1.0, 0.0, 0.0], [2.0**-53, 2.0**-53, 0.0, 0.0], 1.0),  # two ties stay 1 (exact once: 1 + 2^-52)
    ([1.0, 0.0, 0.0, 0.0], [0.75 * E, 0.0, 0.0, 0.0], 1.0),  # above half an ulp: up, not truncated
    ([1.0, 0.0, 0.0, 0.0], [-0.75 * E, 0.0, 0.0, 0.0], -1.0),  # the same, negative
    ([2.0**50, -(2.0**50), 1.0, 0.0], [2.0**50, 2.0**50, 2.0**-60, 0.0], 1.0),  # 1 absorbed, then cancelled
    ([1.0 + E, 0.0, 0.0, 0.0], [1.0 - E / 2, 0.0, 0.0, 0.0], -1.0),  # FMA keeps 2^-53 - 2^-105
    ([1.0, 1.0, 1.0, 1.0], [2.0**-54, 2.0**-54, 2.0**-54, 2.0**-54], 1.0),  # each below half an ulp
    ([3.0, -3.0, 1.0, 1.0], [2.0**60, 2.0**60, 2.0**-53, 2.0**-53], 0.0),  # order: (p0 + p1) first
    ([1.0, 1.0, 0.0, 0.0], [2.0**-53, -(2.0**-53), 0.0, 0.0], 1.0 + E),  # tie to even from odd
]


def run_f64(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    return probe.mfma_f64(t(a), t(b), t(c)).cpu().numpy()


def test_mfma_f64_is_four_fmas_in_k_order_on_crafted_cases() -> None:
    T = len(CASES)
    a = np.zeros((T, 1, 64))
    b = np.zeros((T, 1, 64))
    c = np.zeros((T, 64, 4))
    for t, (ak, bk, ck) in enumerate(CASES):
        for lane in range(64):  # lane l holds A[l % 16][l // 16] and B[l // 16][l % 16]
            a[t, 0, lane], b[t, 0, lane] = ak[lane // 16], bk[lane // 16]
        c[t] = ck  # every output of the tile is the same case
    d = run_f64(a, b, c)
    separated = set()
    for t, (ak, bk, ck) in enumerate(CASES):
        want = fma_chain(ak, bk, ck)
        assert (d[t] == want).all(), (t, d[t, 0, 0].hex(), want.hex())
        exact = sum((Fraction(x) * Fraction(y) for x, y in zip(ak, bk)), Fraction(ck))
        rounded_products = ck
        for x, y in zip(ak, bk):
            rounded_products = rounded_products + x * y
        p = [Fraction(x) * Fraction(y) for x, y in zip(ak, bk)]
        pairwise = float(Fraction(ck) + Fraction(float(Fraction(float(p[0] + p[1])) + Fraction(float(p[2] + p[3])))))
        for name, other in (("exact once", float(exact)), ("rounded products", rounded_products),
                            ("pairwise", pairwise)):  # fmt: skip
            if other != want:
                separated.add(name)
    assert separated == {"exact once", "rounded products", "pairwise"}


def test_mfma_f64_chains_of_random_operands() -> None:
    rng = np.random.default_rng(5)
    tiles = 6
    for steps, kind in ((1, "full"), (4, "full"), (4, "checker")):
        a = rng.standard_normal((tiles, steps, 64)) * np.exp2(rng.integers(-30, 30, (tiles, steps, 64)))
        b = rng.standard_normal((tiles, steps, 64))
        if kind == "checker":  # FP32 bank values times BF16 activations: exact products
            a = a.astype(np.float32).astype(np.float64)
            b = torch.from_numpy(b).to(torch.bfloat16).double().numpy()
        c = rng.standard_normal((tiles, 64, 4)) * 2.0**10
        d = run_f64(a, b, c)
        for t in range(tiles):
            for lane in range(64):
                for v in range(4):
                    i, j = 4 * v + lane // 16, lane % 16  # output layout of the 16 x 16 tile
                    acc = float(c[t, lane, v])
                    for s in range(steps):
                        acc = fma_chain([a[t, s, 16 * k + i] for k in range(4)],
                                        [b[t, s, 16 * k + j] for k in range(4)], acc)  # fmt: skip
                    assert d[t, lane, v] == acc, (kind, steps, t, lane, v)


# ---- BF16 matrix cores ----------------------------------------------------------------------


def bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).float().numpy()


def run_bf16(fn, a: np.ndarray, b: np.ndarray, regs: int) -> np.ndarray:  # type: ignore[no-untyped-def]
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).cuda()  # noqa: E731
    c = torch.zeros((a.shape[0], 64, regs), dtype=torch.float32, device="cuda")
    return fn(t(a), t(b), c).cpu().numpy()


def one_group_operands(rng: np.random.Generator, tiles: int, half: int) -> tuple[np.ndarray, np.ndarray]:
    """(tiles, 1, 64, 8) operands with lane half `half` populated (crafted cases first, then
    random rows of several scales) and the other half zero."""
    rows = []
    for case in crafted():
        pairs = case + [(0.0, 0.0)] * (8 - len(case))
        rows.append(([p[0] for p in pairs], [p[1] for p in pairs]))
    A = np.zeros((tiles * 32, 8), np.float32)
    B = np.zeros((tiles * 32, 8), np.float32)
    for r in range(tiles * 32):
        if r < len(rows):
            A[r], B[r] = rows[r]
        else:
            scale = np.exp2(rng.integers(-40, 40, (2, 8)) * (r % 3 == 0))
            A[r] = rng.standard_normal(8) * scale[0]
            B[r] = rng.standard_normal(8) * scale[1]
    A, B = bf16(A), bf16(B)
    a = np.zeros((tiles, 1, 64, 8), np.float32)
    b = np.zeros((tiles, 1, 64, 8), np.float32)
    a[:, 0, 32 * half : 32 * half + 32] = A.reshape(tiles, 32, 8)
    b[:, 0, 32 * half : 32 * half + 32] = B.reshape(tiles, 32, 8)
    return a, b


@pytest.mark.parametrize("half", [0, 1])
def test_one_group_step_equals_the_oracle(half: int) -> None:
    rng = np.random.default_rng(11 + half)
    tiles = 12
    a, b = one_group_operands(rng, tiles, half)
    d = run_bf16(probe.mfma_bf16, a, b, 16)
    h = 32 * half
    for t in range(tiles):
        lanes = np.arange(64)
        for v in range(16):
            i = 8 * (v // 4) + 4 * (lanes // 32) + v % 4  # output row of lane l, register v
            j = lanes % 32
            want = mfma_step(a[t, 0, h + i], b[t, 0, h + j])
            np.testing.assert_array_equal(d[t, :, v].view(np.uint32), want.view(np.uint32))


def test_nonnegative_16x16x32_step_stays_within_the_checker_bound() -> None:
    rng = np.random.default_rng(21)
    tiles = 32
    scale = np.exp2(rng.integers(-50, 50, (2, tiles, 1, 64, 1)))  # sums stay finite
    a = bf16(np.abs(rng.standard_normal((tiles, 1, 64, 8))) * scale[0] + 2.0**-126)
    b = bf16(np.abs(rng.standard_normal((tiles, 1, 64, 8))) * scale[1] + 2.0**-126)
    d = run_bf16(probe.mfma_bf16_16x16, a, b, 4).astype(np.float64)
    lanes = np.arange(64)
    worst = 0.0
    for t in range(tiles):
        A = np.zeros((16, 32))
        B = np.zeros((16, 32))
        for q in range(4):  # lane l holds row / column l % 16, K slots 8 (l // 16) .. + 7
            A[:, 8 * q : 8 * q + 8] = a[t, 0, 16 * q : 16 * q + 16]
            B[:, 8 * q : 8 * q + 8] = b[t, 0, 16 * q : 16 * q + 16]
        for v in range(4):
            i, j = 4 * (lanes // 16) + v, lanes % 16
            exact = [sum(Fraction(float(x)) * Fraction(float(y)) for x, y in zip(A[r], B[s]))
                     for r, s in zip(i, j)]  # fmt: skip
            for k, ex in enumerate(exact):
                got = Fraction(float(d[t, k, v]))
                floor = ex * (1 - Fraction(1, 2**18)) * (1 - Fraction(1, 2**24)) - 33 * Fraction(1, 2**126)
                assert got >= floor, (t, k, v)
                if ex > 0:
                    worst = max(worst, float((ex - got) / ex))
    print(f"largest relative shortfall of a non-negative step: {worst:.3e}", flush=True)


def _special_nonneg() -> np.ndarray:
    tiny = [0.0, 5e-324, 2.0**-1070, 2.0**-1022, np.nextafter(2.0**-960, 0), 2.0**-960,
            np.nextafter(2.0**-960, 1), 2.0**-700, 2.0**-500, 1e-300]  # fmt: skip
    mid = [2.0**-60, 0.1, 0.75, 1.0, 1.0 + 2.0**-52, 1.5, 3.0, 2.0**52 + 1, 1e100, 2.0**511]
    big = [2.0**600, 1e308, np.finfo(np.float64).max, np.inf, np.nan]
    return np.array(tiny + mid + big, dtype=np.float64)


def _same_bits(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    return (x.view(np.uint64) == y.view(np.uint64)) | (np.isnan(x) & np.isnan(y))


def test_branch_free_round_up_forms_equal_the_general_ones() -> None:
    v = _special_nonneg()
    a, b = (g.ravel() for g in np.meshgrid(v, v, indexing="ij"))
    rng = np.random.default_rng(7)
    ra = np.ldexp(rng.random(4096), rng.integers(-1100, 1000, 4096))
    rb = np.ldexp(rng.random(4096), rng.integers(-1100, 1000, 4096))
    a, b = np.concatenate([a, ra]), np.concatenate([b, rb])
    out = probe.round_up(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()).cpu().numpy()
    print("round-up probe pairs", a.size, flush=True)
    assert _same_bits(out[:, 0], out[:, 1]).all(), np.argwhere(~_same_bits(out[:, 0], out[:, 1]))[:4]
    assert _same_bits(out[:, 2], out[:, 3]).all(), np.argwhere(~_same_bits(out[:, 2], out[:, 3]))[:4]
    with np.errstate(over="ignore", under="ignore"):
        _check_against_exact(a, b, out)


def _check_against_exact(a: np.ndarray, b: np.ndarray, out: np.ndarray) -> None:
    # mul_up against the exact upward product (finite operands)
    for x, y, got in zip(a, b, out[:, 0]):
        if not (np.isfinite(x) and np.isfinite(y)):
            continue
        rn = x * y
        if not np.isfinite(rn):  # beyond the largest double: upward gives +inf
            assert got == np.inf, (x, y, got)
            continue
        exact = Fraction(x) * Fraction(y)
        ru = rn if Fraction(rn) >= exact else np.nextafter(rn, np.inf)
        if exact != 0 and exact < Fraction(2) ** -960:
            assert got in (ru, np.nextafter(ru, np.inf)), (x, y, got, ru)
        else:
            assert got == ru, (x, y, got, ru)
    # add_up against the exact upward sum
    for x, y, got in zip(a, b, out[:, 2]):
        if not (np.isfinite(x) and np.isfinite(y)) or not np.isfinite(x + y):
            continue
        exact = Fraction(x) + Fraction(y)
        rn = x + y
        ru = rn if Fraction(rn) >= exact else np.nextafter(rn, np.inf)
        assert got == ru, (x, y, got, ru)


def test_general_round_up_forms_on_negative_operands() -> None:
    """The general forms also round negative operands upward (the branch-free ones are not
    used there)."""
    rng = np.random.default_rng(8)
    a = np.ldexp(rng.random(2048) - 0.5, rng.integers(-200, 200, 2048))
    b = np.ldexp(rng.random(2048) - 0.5, rng.integers(-200, 200, 2048))
    out = probe.round_up(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()).cpu().numpy()
    for x, y, mul, add in zip(a, b, out[:, 0], out[:, 2]):
        for got, exact, rn in ((mul, Fraction(x) * Fraction(y), x * y), (add, Fraction(x) + Fraction(y), x + y)):
            ru = rn if Fraction(rn) >= exact else np.nextafter(rn, np.inf)
            assert got == ru, (x, y, got, ru)


def test_round_up_under_the_wave_rounding_mode() -> None:
    """add_up_rm2 / add_up_rm4 (one add under the upward mode) give the TwoSum forms' bits, the
    exact upward sum, and leave the mode at round to nearest for the adds after them."""
    v = _special_nonneg()
    a, b = (g.ravel() for g in np.meshgrid(v, v, indexing="ij"))
    rng = np.random.default_rng(9)
    ra = np.ldexp(rng.random(4096), rng.integers(-1100, 1000, 4096))
    rb = np.ldexp(rng.random(4096), rng.integers(-1100, 1000, 4096))
    na = np.ldexp(rng.random(2048) - 0.5, rng.integers(-200, 200, 2048))
    nb = np.ldexp(rng.random(2048) - 0.5, rng.integers(-200, 200, 2048))
    a, b = np.concatenate([a, ra, na]), np.concatenate([b, rb, nb])
    ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    mode = probe.round_up_mode(ta, tb).cpu().numpy()
    twosum = probe.round_up(ta, tb).cpu().numpy()
    print("round-up-mode probe pairs", a.size, flush=True)
    for col in (0, 1):
        assert _same_bits(mode[:, col], twosum[:, 2]).all(), np.argwhere(~_same_bits(mode[:, col], twosum[:, 2]))[:4]
    nonneg = (a >= 0) & (b >= 0)
    assert _same_bits(mode[nonneg, 0], twosum[nonneg, 3]).all()
    with np.errstate(over="ignore", invalid="ignore"):
        rn = a + b
    assert _same_bits(mode[:, 2], rn).all(), np.argwhere(~_same_bits(mode[:, 2], rn))[:4]
    for x, y, got in zip(a, b, mode[:, 0]):
        if not (np.isfinite(x) and np.isfinite(y)) or not np.isfinite(x + y):
            continue
        exact = Fraction(x) + Fraction(y)
        ru = x + y if Fraction(x + y) >= exact else np.nextafter(x + y, np.inf)
        assert got == ru, (x, y, got, ru)
