"""Pins the CPU blocked checker of the oracle (oracle/checker.py).

Mirrors the reference's tests/test_checker.py (theorem mirrors T1, T2, T4, fail-closed
overflow, known verdicts) and reproduces the first table and the false-alarm line of the
reference's recorded harness/sim_out.txt (default_rng(1), 4096 x 4100, naive kernel T = 256).
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
from hypothesis import assume, given
from hypothesis import strategies as st

from oracle.checker import BlockedChecker, WeightBank, gpu_rho_exact, gpu_threshold_exact
from oracle.gemv import abs_row_sums, emulate_gemv, emulate_gemv_coalesced, reference_gemv
from pck.faults import flip_bit
from pck.fp import U32, bf16, gamma, tree_height
from tests.strategies import Problem, gemv_problems

BLOCK = 8


def make_checker(p: Problem, block: int = BLOCK) -> BlockedChecker:
    return BlockedChecker(p.W, p.x, block, tree_height(p.x.size, p.threads))


@given(gemv_problems(row_multiple=BLOCK), st.integers(0, 2**32 - 1))
def test_no_false_alarms_on_legit_kernel(p: Problem, seed: int) -> None:
    """Empirical mirror of T1: a kernel inside the spec never trips the checker."""
    y = emulate_gemv(p.W, p.x, p.threads)
    assert make_checker(p).verdict(y, np.random.default_rng(seed), checks=4).all()


@given(gemv_problems(row_multiple=BLOCK), st.sampled_from([32, 128, 256]), st.integers(0, 2**32 - 1))
def test_no_false_alarms_on_coalesced_kernel(p: Problem, threads: int, seed: int) -> None:
    y = emulate_gemv_coalesced(p.W, p.x, threads)
    checker = BlockedChecker(p.W, p.x, BLOCK, tree_height(p.x.size, threads, vec=8))
    assert checker.verdict(y, np.random.default_rng(seed), checks=4).all()


@given(gemv_problems(row_multiple=BLOCK), st.integers(0, 2**32 - 1), st.data())
def test_large_single_error_always_caught(p: Problem, seed: int, data: st.DataObject) -> None:
    """Empirical mirror of T2: one output off by more than 2 tau fails its block, for any
    signs, and no other block fails."""
    checker = make_checker(p)
    honest = emulate_gemv(p.W, p.x, p.threads)
    y = honest.astype(np.float64)
    i = data.draw(st.integers(0, y.size - 1))
    blk = i // BLOCK
    y[i] += data.draw(st.sampled_from([-1.0, 1.0])) * 2.5 * checker.tau_base[blk]
    y32 = y.astype(np.float32)
    if not np.isfinite(y32).all():
        return
    # the error must survive rounding to FP32 (a threshold of a few FP64 subnormals, as for
    # x = 0, does not)
    assume(abs(float(y32[i]) - float(honest[i])) > 2 * checker.tau_base[blk])
    verdict = checker.verdict(y32, np.random.default_rng(seed), checks=1)
    assert not verdict[blk]
    assert np.delete(verdict, blk).all()


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_non_finite_output_fails_its_block_only(bad: float) -> None:
    rng = np.random.default_rng(0)
    W = bf16(rng.standard_normal((32, 64)) * 0.02)
    x = bf16(rng.standard_normal(64))
    y = emulate_gemv(W, x, 8)
    y[13] = bad
    verdict = BlockedChecker(W, x, BLOCK, tree_height(64, 8)).verdict(y, rng, checks=2)
    np.testing.assert_array_equal(verdict, [True, False, True, True])


@pytest.mark.parametrize("exploit", ["skip_tail", "acc_bf16", "partial_bf16", "bf16_output"])
def test_planted_exploits_caught_at_b64(exploit: str) -> None:
    rng = np.random.default_rng(1)
    m, n, threads = 512, 2048, 128
    W = bf16(rng.standard_normal((m, n)) * 0.02)
    x = bf16(rng.standard_normal(n))
    legit = emulate_gemv(W, x, threads)
    y = {
        "skip_tail": lambda: emulate_gemv(W, x, threads, drop_tail=4),
        "acc_bf16": lambda: emulate_gemv(W, x, threads, acc_bf16=True),
        "partial_bf16": lambda: emulate_gemv(W, x, threads, partial_bf16=True),
        "bf16_output": lambda: bf16(legit),
    }[exploit]()
    checker = BlockedChecker(W, x, 64, tree_height(n, threads))
    assert checker.verdict(legit, rng, checks=8).all()
    assert not checker.verdict(y, rng, checks=8).all()


def test_exponent_flip_to_inf_is_caught() -> None:
    rng = np.random.default_rng(2)
    W = bf16(rng.standard_normal((64, 128)) * 0.02)
    x = bf16(rng.standard_normal(128))
    y = emulate_gemv(W, x, 16)
    y[5] = 1.5  # the top exponent bit set gives Inf/NaN
    flipped = flip_bit(y, 5, 30)
    assert not np.isfinite(flipped[5])
    assert not BlockedChecker(W, x, 64, tree_height(128, 16)).verdict(flipped, rng)[0]


@pytest.mark.parametrize(("block", "x_len", "match"), [(5, 4, "divide"), (0, 4, "positive"), (4, 3, "shape")])
def test_rejects_bad_configuration(block: int, x_len: int, match: str) -> None:
    with pytest.raises(ValueError, match=match):
        BlockedChecker(np.ones((8, 4)), np.ones(x_len), block, 2)


def test_rejects_wrong_output_shape() -> None:
    checker = BlockedChecker(np.ones((8, 4)), np.ones(4), 4, 2)
    with pytest.raises(ValueError, match="shape"):
        checker.verdict(np.ones(7), np.random.default_rng(0))


def test_crafted_output_passes_at_most_half_of_sign_draws() -> None:
    """Empirical mirror of T4: an error that cancels under one guessed sign vector passes at
    most about half of fresh draws."""
    rng = np.random.default_rng(5)
    b, n = 8, 256
    W = bf16(rng.standard_normal((b, n)) * 0.02)
    x = bf16(rng.standard_normal(n))
    checker = BlockedChecker(W, x, b, tree_height(n, 32))
    y = emulate_gemv(W, x, 32).astype(np.float64)
    big = 1.5 * checker.tau_base[0]
    guess = rng.choice([-1.0, 1.0], b)
    y[0] += big
    y[1:] -= guess[0] * big * guess[1:] / (b - 1)
    trials = 2000
    passes = sum(bool(checker.verdict(y.astype(np.float32), rng)[0]) for _ in range(trials))
    assert passes / trials <= 0.5 + 0.04


def test_spread_error_passes_at_most_13_16_of_sign_draws() -> None:
    """T4's Paley-Zygmund part: every output off by less than tau but ||D||_2 >= 2 tau."""
    rng = np.random.default_rng(6)
    b, n = 8, 256
    W = bf16(rng.standard_normal((b, n)) * 0.02)
    x = bf16(rng.standard_normal(n))
    checker = BlockedChecker(W, x, b, tree_height(n, 32))
    y = emulate_gemv(W, x, 32).astype(np.float64)
    tau = checker.tau_base[0]
    D = rng.choice([-1.0, 1.0], b) * (2.05 * tau / np.sqrt(b))
    assert np.all(np.abs(D) < tau) and np.linalg.norm(D) >= 2 * tau
    trials = 2000
    passes = sum(bool(checker.verdict((y + D).astype(np.float32), rng)[0]) for _ in range(trials))
    assert passes / trials <= 13 / 16 + 0.04


def test_an_overflowing_threshold_fails_closed() -> None:
    """Weights of +-2^125 overflow a_beta in FP32; tau = inf must reject, even an honest 0."""
    m, n = 8, 64
    signs = np.where(np.arange(n) % 2 == 0, 1.0, -1.0)
    W = np.tile(signs * 2.0**125, (m, 1)).astype(np.float32)
    checker = BlockedChecker(W, np.ones(n, dtype=np.float32), block=m, height=tree_height(n, 32))
    rng = np.random.default_rng(0)
    assert not checker.verdict(np.full(m, 1e30), rng).any()
    assert not checker.verdict(np.zeros(m), rng).any()


def test_a_shared_weight_bank_gives_the_same_verdicts() -> None:
    rng = np.random.default_rng(1)
    W = bf16(rng.standard_normal((16, 40)))
    bank = WeightBank(W, 8)
    for seed in range(3):
        x = bf16(np.random.default_rng(seed).standard_normal(40))
        y = emulate_gemv(W, x, 4)
        own, shared = BlockedChecker(W, x, 8, 10), BlockedChecker(W, x, 8, 10, bank)
        np.testing.assert_array_equal(own.abs_bound, shared.abs_bound)
        assert (own.verdict(y, np.random.default_rng(0)) == shared.verdict(y, np.random.default_rng(0))).all()
    with pytest.raises(ValueError, match="another W"):
        BlockedChecker(W, x, 16, 10, bank)


def test_explicit_signs_give_the_drawn_verdict() -> None:
    rng = np.random.default_rng(3)
    W = bf16(rng.standard_normal((64, 300)) * 0.02)
    x = bf16(rng.standard_normal(300))
    y = emulate_gemv_coalesced(W, x, 32)
    y[7] += 0.5
    checker = BlockedChecker(W, x, 16, tree_height(300, 32, 8))
    drawn = checker.verdict(y, np.random.default_rng(9), checks=3)
    g = np.random.default_rng(9)
    signs = np.stack([g.choice([-1.0, 1.0], (4, 16)) for _ in range(3)])
    passed, rho, tau = checker.verdict_with_signs(y, signs)
    np.testing.assert_array_equal(passed.all(0), drawn)
    assert not drawn[0] and drawn[1:].all()


def test_gpu_threshold_formula_is_exact_rational() -> None:
    """gpu_threshold_exact equals the formula evaluated by hand in Fractions, and gpu_rho_exact
    equals c.x - r.y to one FP64 rounding."""
    a = np.array([[1.0, 2.0, 0.5]])
    x = np.array([1.0, -2.0, 4.0])
    y = np.array([3.0, -1.0], dtype=np.float32)
    coef, geps, floor = 1e-6, 1e-15, 1e-40
    tau = gpu_threshold_exact(a, x, y, 2, coef, geps, floor)[0]
    s = Fraction(1) + Fraction(4) + Fraction(2)
    expect = Fraction(coef) * s + Fraction(geps) * ((1 + Fraction(U32)) * s + 4) + Fraction(floor)
    assert tau == expect
    c = np.array([[[1.0, 0.5, -0.25]]], dtype=np.float32)
    r = np.array([[[1, -1]]], dtype=np.int8)
    assert gpu_rho_exact(c, r, x, y)[0, 0] == (1 - 1 - 1) - (3 + 1)


@pytest.mark.slow
def test_reproduces_recorded_sim_table_gauss() -> None:
    """harness/sim_out.txt, x ~ gauss (reference harness/numerics_sim.py with default_rng(1)):
    which planted exploits each block size catches with K = 8, the atol = rtol = 1e-2
    comparison, the spec-violation column, and 0 of 12800 false alarms at b = 64, K = 1."""
    rng = np.random.default_rng(1)
    m, n, T = 4096, 4100, 256
    h = tree_height(n, T)
    W = bf16(rng.standard_normal((m, n)) * 0.02)
    x = bf16(rng.standard_normal(n))
    y = reference_gemv(W, x)
    s_row = abs_row_sums(W, x)
    legit = emulate_gemv(W, x, T)
    assert h == 24 and f"{gamma(h):.2e}" == "1.43e-06" and f"{gamma(n - 1):.2e}" == "2.44e-04"
    cases = {
        "legit": legit,
        "skip_tail": emulate_gemv(W, x, T, drop_tail=4),
        "acc_bf16": emulate_gemv(W, x, T, acc_bf16=True),
        "partial_bf16": emulate_gemv(W, x, T, partial_bf16=True),
        "bf16_output": bf16(legit),
    }
    blocks = (8, 64, 128, m)
    checkers = {b: BlockedChecker(W, x, b, h) for b in blocks}
    table = {}
    for name, yk in cases.items():
        e = yk.astype(np.float64) - y
        caught = [not checkers[b].verdict(yk, rng, checks=8).all() for b in blocks]
        kb = bool(np.all(np.abs(e) <= 1e-2 + 1e-2 * np.abs(y)))
        spec = bool(np.any(np.abs(e) > gamma(h) * s_row))
        table[name] = (caught, kb, spec)
    assert table == {
        "legit": ([False] * 4, True, False),
        "skip_tail": ([True] * 4, False, True),
        "acc_bf16": ([True] * 4, False, True),
        "partial_bf16": ([True] * 4, True, True),
        "bf16_output": ([True, True, True, False], True, True),
    }
    c64 = checkers[64]
    alarms = sum(int((~c64.verdict(legit, rng, checks=1)).sum()) for _ in range(200))
    assert alarms == 0  # "false alarms, legit kernel, b=64: 0 of 12800 block checks"
