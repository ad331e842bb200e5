"""pck.fp: the host constants of the path, pinned by known answers, closed forms and exact
arithmetic (mirrors the reference's tests/test_fp.py; ml_dtypes is absent here, so BF16
rounding is checked against torch's own float32 -> bfloat16 conversion instead)."""

from __future__ import annotations

import math
from decimal import Decimal, getcontext
from fractions import Fraction

import numpy as np
import pytest
import torch
from hypothesis import given
from hypothesis import strategies as st

from pck.fp import (
    U32,
    U64,
    bf16,
    ceil_div,
    gamma,
    next_up,
    round_up_f32,
    softmax_eps,
    sum_up,
    sum_up_factor,
    tree_height,
)

f32 = st.floats(width=32, allow_nan=False)
F32_TINY = float(np.finfo(np.float32).tiny)
F32_MAX = float(np.finfo(np.float32).max)
bf16_values = (
    st.floats(width=32, allow_nan=False, allow_infinity=False)
    .map(lambda v: float(bf16(v)))
    .filter(math.isfinite)
)


class TestBf16:
    @pytest.mark.parametrize(
        ("value", "expected"),
        [
            (1.0, 1.0),
            (1 + 2**-8, 1.0),  # tie, to even (down)
            (1 + 3 * 2**-8, 1 + 2**-6),  # tie, to even (up)
            (1 + 2**-8 + 2**-20, 1 + 2**-7),  # just past the tie
            (-1.5, -1.5),
            (0.0, 0.0),
        ],
    )
    def test_known_values(self, value: float, expected: float) -> None:
        assert float(bf16(value)) == expected

    def test_matches_torch_conversion_on_many_bit_patterns(self) -> None:
        """Every finite FP32 pattern in a 2^22 stratified sample (all exponents, both signs,
        the low 16 bits at ties and around them) rounds as torch's RNE cast does."""
        rng = np.random.default_rng(0)
        hi = rng.integers(0, 2**16, 2**22, dtype=np.uint32) << np.uint32(16)
        low = rng.choice(
            np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF], dtype=np.uint32), 2**22
        )
        low = np.where(rng.random(2**22) < 0.5, low, rng.integers(0, 2**16, 2**22, dtype=np.uint32))
        bits = hi | low
        vals = bits.view(np.float32)
        vals = vals[np.isfinite(vals)]
        ours = bf16(vals)
        theirs = torch.from_numpy(vals).to(torch.bfloat16).float().numpy()
        np.testing.assert_array_equal(ours.view(np.uint32), theirs.view(np.uint32))

    @given(f32)
    def test_idempotent_and_low_bits_clear(self, v: float) -> None:
        once = bf16(v)
        assert (once.view(np.uint32) & 0xFFFF) == 0
        assert bf16(once).tobytes() == once.tobytes()

    def test_nan_stays_nan(self) -> None:
        nan = np.array([0x7F800001, 0xFFFFFFFF], dtype=np.uint32).view(np.float32)
        assert np.isnan(bf16(nan)).all()

    def test_overflow_rounds_to_inf(self) -> None:
        assert np.isposinf(bf16(np.finfo(np.float32).max))

    def test_does_not_modify_input(self) -> None:
        a = np.array([1 + 2**-8 + 2**-20], dtype=np.float32)
        before = a.copy()
        bf16(a)
        np.testing.assert_array_equal(a, before)

    @given(bf16_values, bf16_values)
    def test_product_of_two_bf16_is_exact_in_fp32(self, a: float, b: float) -> None:
        """The precision fact the GEMV tree relies on (barring over/underflow)."""
        exact = a * b
        if not (exact == 0 or F32_TINY <= abs(exact) <= F32_MAX):
            return
        assert float(np.float32(a) * np.float32(b)) == exact


class TestGamma:
    def test_zero(self) -> None:
        assert gamma(0) == 0.0

    def test_known_values(self) -> None:
        assert gamma(24) == pytest.approx(24 * U32 / (1 - 24 * U32))
        # the heights of the BASELINE shapes (T = 256): 23, 63 (BF16 down), 71 (FP8 down)
        assert f"{gamma(23):.3e}" == "1.371e-06"
        assert f"{gamma(63):.3e}" == "3.755e-06"
        assert f"{gamma(71):.3e}" == "4.232e-06"

    @given(st.integers(0, 10**6))
    def test_increasing_and_above_ku(self, k: int) -> None:
        assert gamma(k + 1) > gamma(k) >= k * U32

    def test_exact_value(self) -> None:
        for k in (1, 23, 4097):
            exact = Fraction(k) * Fraction(U32) / (1 - Fraction(k) * Fraction(U32))
            assert abs(Fraction(gamma(k)) - exact) <= exact * Fraction(2, 2**53)

    def test_rejects_ku_at_least_one(self) -> None:
        with pytest.raises(ValueError, match="k\\*u < 1"):
            gamma(2**24)

    def test_rejects_negative(self) -> None:
        with pytest.raises(ValueError, match="non-negative"):
            gamma(-1)


class TestRoundUpF32:
    @given(st.floats(0, F32_MAX, allow_nan=False))
    def test_never_rounds_down_and_is_tight(self, v: float) -> None:
        up = float(round_up_f32(np.array([v]))[0])
        assert up >= v
        assert float(np.float32(up)) == up
        below = float(np.nextafter(np.float32(up), np.float32(0)))
        assert below < v or up == 0

    def test_rejects_negative(self) -> None:
        with pytest.raises(ValueError, match="non-negative"):
            round_up_f32(np.array([-1.0]))


class TestTreeHeight:
    @pytest.mark.parametrize(
        ("n", "threads", "expected"),
        [(4100, 256, 24), (4096, 256, 23), (1, 1, 0), (5, 1, 4), (3, 8, 3)],
    )
    def test_known_values(self, n: int, threads: int, expected: int) -> None:
        assert tree_height(n, threads) == expected

    @pytest.mark.parametrize(
        ("n", "threads", "vec", "expected"),
        [
            (4096, 256, 8, 23),
            (4100, 256, 8, 31),
            (4096, 128, 8, 38),
            (1, 32, 8, 12),
            (14336, 256, 8, 63),
            (4096, 256, 16, 23),
            (14336, 256, 16, 71),
        ],
    )
    def test_vectorized_known_values(self, n: int, threads: int, vec: int, expected: int) -> None:
        assert tree_height(n, threads, vec) == expected

    @given(st.integers(1, 10**5), st.integers(0, 10), st.integers(1, 16))
    def test_formula(self, n: int, log_t: int, vec: int) -> None:
        t = 2**log_t
        chain = vec * math.ceil(math.ceil(n / vec) / t)
        assert tree_height(n, t, vec) == chain - 1 + log_t

    @pytest.mark.parametrize("threads", [0, 3, 6, -2])
    def test_rejects_non_power_of_two(self, threads: int) -> None:
        with pytest.raises(ValueError, match="power of two"):
            tree_height(10, threads)

    def test_rejects_empty_and_bad_vec(self) -> None:
        with pytest.raises(ValueError, match="positive"):
            tree_height(0, 4)
        with pytest.raises(ValueError, match="vec"):
            tree_height(10, 4, 0)


@given(st.integers(0, 10**9), st.integers(1, 10**6))
def test_ceil_div(a: int, b: int) -> None:
    assert ceil_div(a, b) == math.ceil(Fraction(a, b))


def test_next_up_steps() -> None:
    assert next_up(1.0) == 1.0 + 2.0**-52
    assert next_up(1.0, 2) == 1.0 + 2.0**-51
    assert next_up(0.0) == 5e-324


@given(st.lists(st.floats(0, 1e300), min_size=1, max_size=200))
def test_sum_up_bounds_the_exact_sum(values: list[float]) -> None:
    """`sum_up` of a round-to-nearest sum is never below the exact sum, in any order."""
    exact = sum(Fraction(v) for v in values)
    for order in (values, values[::-1], sorted(values)):
        s = 0.0
        for v in order:
            s += v
        assert Fraction(float(sum_up(s, len(values)))) >= exact


def test_sum_up_factor_value() -> None:
    assert sum_up_factor(128) == next_up(1.0 + 2.0 * gamma(128, U64))
    assert sum_up_factor(0) == sum_up_factor(1)


def _softmax_mass64(logits: np.ndarray, sel: np.ndarray, temperature: float) -> float:
    z = logits.astype(np.float64) / temperature
    e = np.exp(z - z.max())
    return float((e / e.sum())[sel].sum())


@given(
    st.lists(st.floats(-50, 50), min_size=2, max_size=60),
    st.sampled_from([1.0, 0.7, 0.01]),
    st.data(),
)
def test_softmax_eps_bounds_the_fp64_softmax_mass(
    logits: list[float], temperature: float, data: st.DataObject
) -> None:
    """An FP64 softmax mass stays within `softmax_eps` of the exact one (60-digit Decimal)."""
    getcontext().prec = 60
    a = np.array(logits, dtype=np.float32)
    k = data.draw(st.integers(1, a.size))
    sel = np.argsort(-a.astype(np.float64), kind="stable")[:k]
    z = [Decimal(float(v)) / Decimal(temperature) for v in a]
    top = max(z)
    e = [(v - top).exp() for v in z]
    exact = sum(e[i] for i in sel) / sum(e)
    computed = _softmax_mass64(a, sel, temperature)
    zmax = 0.0 if temperature == 1.0 else float(np.abs(a.astype(np.float64) / temperature).max())
    assert abs(Decimal(computed) - exact) <= Decimal(softmax_eps(a.size, zmax))


def test_softmax_eps_refuses_unrepresentable_ranges() -> None:
    with pytest.raises(ValueError, match="too large"):
        softmax_eps(10, zmax=1e15)
