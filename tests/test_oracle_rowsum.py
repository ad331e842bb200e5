"""Pins of the in-pass checksum oracle (`oracle.rowsum`), independent of the GPU.

- row sums: exact for small integers (any order gives the exact sum), within their bounds of
  the exact rational sums for random BF16 and E4M3 data, and hand-worked cases whose values
  depend on the lane order (the documented order gives 0, a sequential sum 7) and on the pairs
  being rounded in FP32;
- the check's threshold is never below the exact rational threshold and at most 2^-14 above
  it; rho is within u32 S + geps (S + sum |y|) of the exact r^T (W x - y);
- its verdicts equal the CPU bank checker's (`oracle.checker.BlockedChecker`, same signs) on
  honest and faulty outputs wherever |rho| is clear of both thresholds, whose values agree to
  2^-14 (the CPU checker's a is FP32 rounded up, as tight as the exact s);
- the directed-rounding helpers against exact rationals.
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest

from oracle.checker import BlockedChecker
from oracle.gemv import e4m3_values, emulate_gemv, emulate_gemv_coalesced
from oracle.rowsum import (
    add_up,
    add_up_nonneg,
    depth_of,
    exact_rho,
    exact_rowsum_threshold,
    mul_up,
    mul_up_nonneg,
    row_sums,
    rowsum_check_with_signs,
    rowsum_constants,
    up_to_f32,
)
from pck.fp import U32, U64, bf16, gamma, tree_height


def test_integer_row_sums_are_exact() -> None:
    rng = np.random.default_rng(0)
    W = rng.integers(-8, 9, (17, 300)).astype(np.float64)
    x = rng.integers(-4, 5, 300).astype(np.float64)
    for threads, vec in ((32, 8), (256, 8), (1024, 16)):
        got = row_sums(W, x, threads, vec)
        assert np.array_equal(got[:, 0], W @ x)
        assert np.array_equal(got[:, 1], np.abs(W) @ np.abs(x))


@pytest.mark.parametrize("vec", [8, 16])
def test_row_sums_within_their_bounds(vec: int) -> None:
    """d within u32 S (the FP32 pair sums) + gamma_D(u64) S of the exact W x; s within
    gamma_D(u32) of S, and s_factor s >= S."""
    rng = np.random.default_rng(vec)
    n = 700
    if vec == 16:
        W = e4m3_values()[rng.integers(0, 256, (6, n))]
        W[~np.isfinite(W)] = 0.0
    else:
        W = bf16(rng.standard_normal((6, n)) * 0.02).astype(np.float64)
    x = bf16(rng.standard_normal(n)).astype(np.float64)
    got = row_sums(W, x, 256, vec)
    D = depth_of(n, 256, vec)
    F = rowsum_constants(n, 128, 23)["s_factor"]
    for i in range(6):
        exact = sum((Fraction(float(w)) * Fraction(float(v)) for w, v in zip(W[i], x)), Fraction(0))
        S = sum((abs(Fraction(float(w)) * Fraction(float(v))) for w, v in zip(W[i], x)), Fraction(0))
        assert abs(Fraction(float(got[i, 0])) - exact) <= (Fraction(U32) + Fraction(gamma(D, U64))) * S
        assert Fraction(float(got[i, 1])) * Fraction(F) >= S
        assert abs(Fraction(float(got[i, 1])) - S) <= Fraction(gamma(D, U32)) * S


def test_pairs_are_rounded_in_fp32() -> None:
    # products 1 and 2^-30 (columns 0, 1: one pair) then 2^-30 and -1 (columns 2, 3): in FP32
    # each pair sum rounds to +-1, so d = 0 (an FP64 sum of the products would give 2^-29)
    W = np.zeros((1, 8))
    x = np.ones(8)
    W[0, :4] = [1.0, 2.0**-30, 2.0**-30, -1.0]
    assert row_sums(W, x, 256, 8)[0, 0] == 0.0


def test_depth_matches_the_tree() -> None:
    # n = 4096, T = 256, V = 8: lane l runs 4 chains of 2 positions of 8 columns (64 terms),
    # then 6 butterfly levels; T = 32: one chain of 16 positions (128 terms) and 5 levels.
    assert depth_of(4096, 256, 8) == 70
    assert depth_of(4096, 32, 8) == 133
    assert depth_of(14336, 1024, 16) == 16 * 16 + 6
    from pck.cuda.checker import rowsum_depth  # the product's own computation

    for n in (1, 8, 40, 4096, 4100, 14336, 100000):
        assert rowsum_depth(n) == max(
            depth_of(n, t, v) for t in (32, 64, 128, 256, 512, 1024) for v in (8, 16)
        )


def test_lane_order_hand_case() -> None:
    # threads = 32, vec = 8, n = 16: lane 0 owns columns 0-7, lane 1 columns 8-15, lanes 2-31
    # only padding.  Products: lane 0 [2^60, 1 x 7], lane 1 [-2^60, 1 x 7].  Lane 0's d ends on
    # 2^60 (its pair sums 2^60, 2, 2, 2 each add less than half an ulp of 2^60 in FP64), lane
    # 1's on -2^60, and the butterfly's last step gives 0.  Column order (2^60 + 1 ... - 2^60
    # + 1 ...) would give 7, the exact sum 14.  s: 2^60 per lane in FP32, 2^61 in total.
    W = np.ones((1, 16))
    x = np.ones(16)
    W[0, 0], x[0] = 2.0**30, 2.0**30
    W[0, 8], x[8] = -(2.0**30), 2.0**30
    got = row_sums(W, x, 32, 8)
    assert got[0, 0] == 0.0
    assert got[0, 1] == 2.0**61


def test_rounding_helpers_against_rationals() -> None:
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.standard_normal(200) * 10.0 ** rng.integers(-30, 30, 200),
                           [0.0, 5e-324, 1e-310, 1.0, 2.0**-970]])  # fmt: skip
    for a, b in zip(vals[::2], vals[1::2]):
        a, b = float(a), float(b)
        s = add_up(a, b)
        assert Fraction(s) >= Fraction(a) + Fraction(b)
        assert s <= math.nextafter(math.nextafter(a + b, math.inf), math.inf)
        p = mul_up(a, b)
        assert Fraction(p) >= Fraction(a) * Fraction(b)
        aa, bb = abs(a), abs(b)
        assert Fraction(add_up_nonneg(aa, bb)) >= Fraction(aa) + Fraction(bb)
        assert Fraction(mul_up_nonneg(aa, bb)) >= Fraction(aa) * Fraction(bb)
    assert up_to_f32(1.0 + 2.0**-30) == float(np.nextafter(np.float32(1), np.float32(2)))
    assert up_to_f32(1.0) == 1.0
    assert up_to_f32(3.5e38) == math.inf


def honest_and_faulty(seed: int, m: int = 512, n: int = 512):  # type: ignore[no-untyped-def]
    rng = np.random.default_rng(seed)
    W = bf16(rng.standard_normal((m, n), dtype=np.float32) * np.float32(0.02))
    x = bf16(rng.standard_normal(n, dtype=np.float32))
    y = emulate_gemv_coalesced(W, x, 256)
    faults = {
        "drop_tail": emulate_gemv(W, x, 256, drop_tail=4),
        "bf16_accumulator": emulate_gemv(W, x, 256, acc_bf16=True),
        "bf16_output": bf16(y).astype(np.float32),
        "bump": y + np.float32(0.05) * (np.arange(m) % 128 == 3),
    }
    return W, x, y, faults


def test_threshold_and_rho_against_exact() -> None:
    W, x, y, faults = honest_and_faulty(2, m=256, n=256)
    block, h = 128, tree_height(256, 256, 8)
    c = rowsum_constants(256, block, h)
    signs = np.where(np.random.default_rng(3).integers(0, 2, (2, 2, block)) > 0, 1, -1)
    sums = row_sums(W.astype(np.float64), x.astype(np.float64), 256, 8)
    for yy in (y, faults["bf16_output"]):
        passed, rho, tau = rowsum_check_with_signs(sums, yy, signs, block, **c)
        exact_tau = exact_rowsum_threshold(W, x, yy, block, c["coef"], c["geps"], c["tau_floor"])
        ex_rho = exact_rho(W, x, yy, signs, block)
        for beta in range(2):
            for k in range(2):
                assert Fraction(tau[k, beta]) >= exact_tau[beta]
                assert Fraction(tau[k, beta]) <= exact_tau[beta] * (1 + Fraction(1, 2**14))
                Y = sum((abs(Fraction(float(v))) for v in yy[beta * 128 : (beta + 1) * 128]), Fraction(0))
                S = (exact_tau[beta] - Fraction(c["tau_floor"]) - Fraction(c["geps"]) * Y) / (
                    Fraction(c["coef"]) + Fraction(c["geps"]) * (1 + Fraction(2**-24))
                )
                # the FP32 pair sums (u32 S, inside coef's budget) plus the FP64 evaluation
                bound = Fraction(U32) * S + Fraction(c["geps"]) * (S + Y)
                assert abs(Fraction(rho[k, beta]) - ex_rho[k][beta]) <= bound


@pytest.mark.parametrize("seed", [4, 5])
def test_verdicts_equal_cpu_bank_checker(seed: int) -> None:
    W, x, y, faults = honest_and_faulty(seed)
    block, h = 128, tree_height(512, 256, 8)
    c = rowsum_constants(512, block, h)
    signs = np.where(np.random.default_rng(seed).integers(0, 2, (1, 4, block)) > 0, 1, -1)
    sums = row_sums(W.astype(np.float64), x.astype(np.float64), 256, 8)
    bank = BlockedChecker(W, x, block, h)
    caught = {}
    for name, yy in {"honest": y, **faults}.items():
        pa, rho_a, tau_a = bank.verdict_with_signs(yy, signs.astype(np.float64))
        pb, rho_b, tau_b = rowsum_check_with_signs(sums, yy, signs, block, **c)
        # the CPU checker keeps a in FP32 rounded up, so both thresholds bound the same exact
        # quantity to within a few ulps
        assert (np.abs(tau_b - tau_a) <= 2.0**-14 * tau_a).all()
        lo, hi = np.minimum(tau_a, tau_b), np.maximum(tau_a, tau_b)
        clear = (np.abs(rho_a) < 0.99 * lo) | (np.abs(rho_a) > 1.01 * hi)
        assert np.array_equal(pa[clear], pb[clear]), name
        caught[name] = not pb.all()
    assert caught == {"honest": False, "drop_tail": True, "bf16_accumulator": True,
                      "bf16_output": caught["bf16_output"], "bump": True}  # fmt: skip


def test_non_finite_output_fails_its_block() -> None:
    W, x, y, _ = honest_and_faulty(6, m=256, n=256)
    c = rowsum_constants(256, 128, 23)
    sums = row_sums(W.astype(np.float64), x.astype(np.float64), 256, 8)
    signs = np.ones((1, 2, 128), dtype=np.int64)
    yy = y.copy()
    yy[200] = np.nan
    passed, _, _ = rowsum_check_with_signs(sums, yy, signs, 128, **c)
    assert passed.tolist() == [[True, False]]
