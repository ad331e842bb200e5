"""The CPU set checker (`oracle/sampling.py`) pinned against the reference's known answers and
properties (`tests/test_sampling.py` of proof-carrying-kernels), a closed form for uniform
logits, and brute force over every subset of small vocabularies; `pck.faults.sharded_topk`
against its documented behaviour."""

from __future__ import annotations

import itertools

import numpy as np
import pytest
from hypothesis import assume, given, settings
from hypothesis import strategies as st
from numpy.typing import NDArray

from oracle.sampling import (
    check_sampled,
    check_topk,
    check_topp,
    softmax64,
    topk_reference,
    topp_reference,
)
from pck.faults import sharded_topk
from pck.fp import bf16


@st.composite
def logit_vectors(draw: st.DrawFn, max_size: int = 300) -> NDArray[np.float32]:
    """Seeded normal logits at several scales; BF16 rounding of some draws makes ties."""
    size = draw(st.integers(1, max_size))
    rng = np.random.default_rng(draw(st.integers(0, 2**32 - 1)))
    a = (rng.standard_normal(size) * draw(st.sampled_from([0.1, 1.0, 5.0, 30.0]))).astype(np.float32)
    return bf16(a) if draw(st.booleans()) else a


# ---- known answers (reference tests/test_sampling.py:51-70, 104-121, 124-127) ----------------


def test_ties_may_go_either_way() -> None:
    a = np.array([3.0, 1.0, 2.0, 2.0], dtype=np.float32)
    assert check_topk(a, [0, 2], 2) and check_topk(a, [0, 3], 2)
    assert not check_topk(a, [0, 1], 2)


@pytest.mark.parametrize("selected", [[0, 0], [0, 4], [-1, 0], [0], [0, 1, 2], [], [0.0, 1.0], [[0, 1]]])
def test_malformed_selection_fails(selected: list[object]) -> None:
    assert not check_topk(np.array([4.0, 3.0, 2.0, 1.0], dtype=np.float32), np.asarray(selected), 2)


def test_nan_and_select_all() -> None:
    assert not check_topk(np.array([4.0, np.nan, 2.0], dtype=np.float32), [0, 2], 2)
    assert check_topk(np.array([1.0, 2.0], dtype=np.float32), [1, 0], 2)


def test_topp_non_prefix_and_duplicates_fail() -> None:
    a = np.array([5.0, 4.0, 0.0], dtype=np.float32)
    assert check_topp(a, [0, 1], 0.99)
    assert not check_topp(a, [0, 2], 0.99)
    assert not check_topp(np.array([1.0, 2.0], dtype=np.float32), [1, 1], 0.5)


def test_bad_arguments() -> None:
    a = np.array([1.0, 2.0], dtype=np.float32)
    with pytest.raises(ValueError, match="p must"):
        check_topp(a, [1], 0.0)
    with pytest.raises(ValueError, match="tol"):
        check_topp(a, [1], 0.5, tol=-1.0)
    with pytest.raises(ValueError, match="p must"):
        topp_reference(a, 1.5)
    with pytest.raises(ValueError, match="temperature"):
        softmax64(a, 0.0)
    with pytest.raises(ValueError, match="k must"):
        topk_reference([1.0, 2.0], 3)
    with pytest.raises(ValueError, match="non-empty"):
        topk_reference([], 1)
    with pytest.raises(ValueError, match="per_shard"):
        sharded_topk(np.ones(4, np.float32), 2, 2, 0)


def test_sampled_token_membership() -> None:
    assert check_sampled(3, [1, 3, 5]) and not check_sampled(2, [1, 3, 5])


# ---- properties (reference tests/test_sampling.py:33-49, 73-103, 131-161) ---------------------


@given(logit_vectors(), st.data())
def test_topk_reference_passes(a: NDArray[np.float32], data: st.DataObject) -> None:
    k = data.draw(st.integers(1, a.size))
    assert check_topk(a, topk_reference(a, k), k)


@given(logit_vectors(), st.data())
def test_swapping_in_the_smallest_rejected_fails_unless_tied(a: NDArray[np.float32], data: st.DataObject) -> None:
    assume(a.size >= 2)
    k = data.draw(st.integers(1, a.size - 1))
    sel = topk_reference(a, k)
    rejected = np.setdiff1d(np.arange(a.size), sel)
    worst, best = rejected[np.argmin(a[rejected])], sel[np.argmax(a[sel])]
    assert check_topk(a, np.where(sel == best, worst, sel), k) == (a[worst] == a[best])


@given(logit_vectors(), st.floats(0.01, 1.0), st.sampled_from([0.5, 1.0, 2.0]))
def test_topp_reference_passes(a: NDArray[np.float32], p: float, temp: float) -> None:
    assert check_topp(a, topp_reference(a, p, temp), p, temp, tol=0.0)


@given(logit_vectors(), st.floats(0.05, 0.95), st.sampled_from([0.7, 1.0]))
def test_fp32_softmax_sampler_passes_with_its_tolerance(a: NDArray[np.float32], p: float, temp: float) -> None:
    z = a / np.float32(temp)
    e = np.exp(z - z.max())
    probs32 = (e / e.sum()).astype(np.float32)
    order = np.lexsort((np.arange(a.size), -a.astype(np.float64)))
    count = min(int(np.searchsorted(np.cumsum(probs32[order], dtype=np.float32), np.float32(p))) + 1, a.size)
    assert check_topp(a, order[:count], p, temp, tol=1e-5)


@given(logit_vectors(), st.floats(0.05, 0.9))
def test_one_token_too_many_or_too_few(a: NDArray[np.float32], p: float) -> None:
    sel = topp_reference(a, p)
    probs = softmax64(a)
    order = np.lexsort((np.arange(a.size), -a.astype(np.float64)))
    if sel.size < a.size and abs(probs[sel].sum() - p) > 1e-12:
        assert check_topp(a, order[: sel.size + 1], p, tol=0.0) == (probs[sel].sum() < p)
    if sel.size > 1 and abs(probs[order[: sel.size - 1]].sum() - p) > 1e-12:
        assert check_topp(a, order[: sel.size - 1], p, tol=0.0) == (probs[order[: sel.size - 1]].sum() >= p)


@given(logit_vectors(), st.data())
def test_sharded_topk_exact_with_enough_per_shard(a: NDArray[np.float32], data: st.DataObject) -> None:
    k = data.draw(st.integers(1, a.size))
    assert check_topk(a, sharded_topk(a, k, data.draw(st.integers(1, 8)), per_shard=k), k)


@given(logit_vectors(), st.data())
def test_checker_catches_every_wrong_sharded_set(a: NDArray[np.float32], data: st.DataObject) -> None:
    k = data.draw(st.integers(1, a.size))
    got = sharded_topk(a, k, data.draw(st.integers(1, 8)), data.draw(st.integers(1, k)))
    wrong = got.size != k or not np.array_equal(np.sort(a[got])[::-1], np.sort(a)[::-1][:k])
    assert check_topk(a, got, k) == (not wrong)


def test_clustered_top_logits_are_missed() -> None:
    a = np.zeros(64, dtype=np.float32)
    a[:4] = [9.0, 8.0, 7.0, 6.0]  # all in the first of 8 shards
    assert not check_topk(a, sharded_topk(a, 4, shards=8, per_shard=2), 4)


# ---- closed form and brute force ---------------------------------------------------------------


@pytest.mark.parametrize("vocab", [7, 100, 1000])
def test_uniform_logits_nucleus_size(vocab: int) -> None:
    """Equal logits have mass i / V after i tokens, so p = (j + 1/2) / V needs j + 1 tokens."""
    a = np.full(vocab, 0.25, np.float32)
    for j in (0, vocab // 3, vocab - 1):
        p = (j + 0.5) / vocab
        sel = topp_reference(a, p)
        assert sel.size == j + 1
        assert check_topp(a, sel, p, tol=0.0)
        if j:
            assert not check_topp(a, sel[:-1], p, tol=0.0)
        if j + 1 < vocab:
            assert not check_topp(a, np.arange(j + 2), p, tol=0.0)


@settings(max_examples=40, deadline=None)
@given(st.integers(1, 6), st.integers(0, 2**32 - 1), st.floats(0.05, 0.95))
def test_brute_force_over_every_subset(vocab: int, seed: int, p: float) -> None:
    """check_topk and check_topp against their definitions evaluated subset by subset: a set
    is top-k when it has k members none smaller than a non-member; it is a minimal top-p
    nucleus when it is such a prefix whose mass reaches p and whose mass without its smallest
    member does not (cases within 1e-9 of p are skipped)."""
    rng = np.random.default_rng(seed)
    a = bf16(rng.standard_normal(vocab).astype(np.float32) * 2)  # ties from BF16 rounding
    probs = softmax64(a)
    for size in range(1, vocab + 1):
        for sub in itertools.combinations(range(vocab), size):
            rest = [j for j in range(vocab) if j not in sub]
            prefix = all(a[i] >= a[j] for i in sub for j in rest)
            for k in range(1, vocab + 1):
                assert check_topk(a, np.array(sub), k) == (prefix and size == k)
            mass = sum(float(probs[i]) for i in sub)
            smallest = min(sub, key=lambda i: (a[i], -i))
            without = mass - float(probs[smallest])
            if abs(mass - p) < 1e-9 or abs(without - p) < 1e-9:
                continue
            assert check_topp(a, np.array(sub), p, tol=0.0) == (prefix and mass >= p and without < p)
