"""The reference's CPU API as this package exports it (`pck.emulate_gemv*`, `pck.BlockedChecker`,
`pck.sampling`, `pck.member.check_member`), against the test oracle's independent
restatements on the same inputs: bit-identical model outputs, identical verdicts, equal
selections, and the names of the reference's `pck/__init__.py`."""

from __future__ import annotations

import math

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

import pck
from oracle import checker as ochecker
from oracle import gemv as ogemv
from oracle import member as omember
from oracle import sampling as osampling
from pck import checker as pchecker
from pck import gemv as pgemv
from pck import member as pmember
from pck import sampling as psampling
from pck.fp import bf16, tree_height
from tests.strategies import Problem, gemv_problems


def bits(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def test_top_level_names_of_the_reference() -> None:
    for name in ("U32", "U64", "WARP", "BlockedChecker", "abs_row_sums", "bf16", "ceil_div",
                 "emulate_gemv", "emulate_gemv_coalesced", "flip_bit", "gamma", "reference_gemv",
                 "round_up_f32", "tree_height"):  # fmt: skip
        assert name in pck.__all__ and hasattr(pck, name), name
    assert pck.WARP == ogemv.WARP == 32


@settings(max_examples=60, deadline=None)
@given(gemv_problems(), st.sampled_from([1, 2, 8, 32, 256]), st.sampled_from(["none", "acc", "partial", "tail"]))
def test_naive_model_equals_the_oracle(p: Problem, threads: int, shortcut: str) -> None:
    kw = {"acc": {"acc_bf16": True}, "partial": {"partial_bf16": True},
          "tail": {"drop_tail": min(4, p.x.size)}}.get(shortcut, {})  # fmt: skip
    got = pgemv.emulate_gemv(p.W, p.x, threads, **kw)
    np.testing.assert_array_equal(bits(got), bits(ogemv.emulate_gemv(p.W, p.x, threads, **kw)))


@settings(max_examples=60, deadline=None)
@given(gemv_problems(), st.sampled_from([32, 64, 256, 1024]), st.sampled_from([1, 8, 16]))
def test_coalesced_model_equals_the_oracle(p: Problem, threads: int, vec: int) -> None:
    got = pgemv.emulate_gemv_coalesced(p.W, p.x, threads, vec)
    want = ogemv.emulate_gemv_coalesced(p.W, p.x, threads, vec)
    np.testing.assert_array_equal(bits(got), bits(want))


def test_fp64_helpers_and_argument_checks() -> None:
    rng = np.random.default_rng(1)
    W, x = bf16(rng.standard_normal((9, 300))), bf16(rng.standard_normal(300))
    np.testing.assert_array_equal(pgemv.reference_gemv(W, x), ogemv.reference_gemv(W, x))
    np.testing.assert_array_equal(pgemv.abs_row_sums(W, x), ogemv.abs_row_sums(W, x))
    a = rng.standard_normal((3, 64)).astype(np.float32)
    np.testing.assert_array_equal(bits(pgemv.halving_sum(a)), bits(ogemv.halving_sum(a)))
    with pytest.raises(ValueError, match="power of two"):
        pgemv.emulate_gemv(W, x, 3)
    with pytest.raises(ValueError, match=">= 32"):
        pgemv.emulate_gemv_coalesced(W, x, 16)
    with pytest.raises(ValueError, match="shape"):
        pgemv.emulate_gemv_coalesced(W, x[:10], 32)


@pytest.mark.parametrize("shortcut", ["honest", "acc", "partial", "tail", "flip"])
def test_blocked_checker_verdicts_equal_the_oracle(shortcut: str) -> None:
    rng = np.random.default_rng(3)
    m, n, block, threads = 64, 1000, 8, 32
    W, x = bf16(rng.standard_normal((m, n)) * 0.02), bf16(rng.standard_normal(n))
    kw = {"acc": {"acc_bf16": True}, "partial": {"partial_bf16": True},
          "tail": {"drop_tail": 4}}.get(shortcut, {})  # fmt: skip
    y = pgemv.emulate_gemv(W, x, threads, **kw)
    if shortcut == "flip":
        y = y.copy()
        y.view(np.uint32)[5] ^= np.uint32(1 << 30)
    height = tree_height(n, threads)
    mine = pchecker.BlockedChecker(W, x, block, height)
    ref = ochecker.BlockedChecker(W, x, block, height)
    np.testing.assert_array_equal(mine.tau_base, ref.tau_base)
    got = mine.verdict(y, np.random.default_rng(11), checks=3)
    np.testing.assert_array_equal(got, ref.verdict(y, np.random.default_rng(11), checks=3))
    if shortcut == "honest":
        assert got.all()
    bank = pchecker.WeightBank(W, block)
    np.testing.assert_array_equal(pchecker.BlockedChecker(W, x, block, height, bank=bank).verdict(
        y, np.random.default_rng(11), checks=3), got)  # fmt: skip
    y_nan = y.copy()
    y_nan[13] = np.nan
    assert not mine.verdict(y_nan, np.random.default_rng(0))[13 // block]
    with pytest.raises(ValueError, match="divide"):
        pchecker.WeightBank(W, 7)


def sampling_cases() -> list[tuple[np.ndarray, np.ndarray]]:
    rng = np.random.default_rng(5)
    cases = []
    for v in (1, 2, 7, 50, 1000):
        a = (rng.standard_normal(v) * 3).astype(np.float32)
        order = np.argsort(-a, kind="stable")
        for k in {1, max(1, v // 3), v}:
            cases.append((a, order[:k].copy()))
        cases.append((a, order[1 : max(2, v // 2)].copy()))  # not a prefix
        cases.append((a, np.array([0, 0])))  # repeated index
        cases.append((a, np.array([v])))  # out of range
        cases.append((a, np.array([0.0])))  # not integers
    tied = np.array([1.0, 2.0, 2.0, 2.0, 0.5], dtype=np.float32)
    cases += [(tied, np.array([1, 2])), (tied, np.array([3, 1])), (tied, np.array([1, 2, 3]))]
    nan = np.array([1.0, np.nan, 0.0], dtype=np.float32)
    cases.append((nan, np.array([0])))
    return cases


def test_sampling_checks_equal_the_oracle() -> None:
    for a, sel in sampling_cases():
        for k in (1, 2, 3, len(sel)):
            assert psampling.check_topk(a, sel, k) == osampling.check_topk(a, sel, k)
        for p in (0.1, 0.5, 0.9, 1.0):
            for t in (1.0, 0.7):
                assert psampling.check_topp(a, sel, p, t, 1e-6) == osampling.check_topp(a, sel, p, t, 1e-6)
        for token in (0, 1, len(a)):
            assert psampling.check_sampled(token, sel) == osampling.check_sampled(token, sel)


def test_reference_samplers_equal_the_oracle() -> None:
    rng = np.random.default_rng(8)
    for v in (1, 5, 300, 5000):
        a = (rng.standard_normal(v) * 2).astype(np.float32)
        a[rng.integers(0, v, v // 4)] = a[0]  # ties
        np.testing.assert_array_equal(psampling.softmax64(a, 0.8), osampling.softmax64(a, 0.8))
        for k in {1, max(1, v // 10), v}:
            np.testing.assert_array_equal(psampling.topk_reference(a, k), osampling.topk_reference(a, k))
        for p in (0.05, 0.5, 0.95, 1.0):
            np.testing.assert_array_equal(psampling.topp_reference(a, p, 1.3), osampling.topp_reference(a, p, 1.3))
            sel = psampling.topp_reference(a, p)
            assert psampling.check_topp(a, sel, p) and psampling.check_topk(a, sel, sel.size)


def same(a: float, b: float) -> bool:
    return a == b or (math.isnan(a) and math.isnan(b))


def test_check_member_equals_the_oracle() -> None:
    rng = np.random.default_rng(9)
    for trial in range(300):
        v = int(rng.choice([1, 3, 50, 2000]))
        row = (rng.standard_normal(v) * 3).astype(np.float32)
        if trial % 25 == 0:
            row[rng.integers(0, v)] = np.nan
        token = int(rng.integers(-1, v + 1))
        top_k = [None, 1, 5, v][trial % 4]
        top_p = [None, 0.5, 0.9, 1.0][(trial // 4) % 4]
        greedy = trial % 7 == 0
        got = pmember.check_member(row, token, top_k, top_p, greedy=greedy, tol=1e-4)
        want = omember.check_member(row, token, top_k, top_p, greedy=greedy, tol=1e-4)
        assert (got.ok, got.above) == (want.ok, want.above) and same(got.mass_above, want.mass_above)
