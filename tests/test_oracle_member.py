"""Pins the membership oracle (oracle/member.py) and pck.member's error bounds.

Mirrors the reference's tests/test_member.py: brute-force equivalence of the top-k rule with
"t is in some correct top-k set", every token vLLM's own masking keeps is accepted (no false
alarms), hand cases, the bound magnitudes, and the batched semantics (top-(max k) path, ties,
stale host copy, bad ids) against the per-row FP64 reference.  mpmath checks the FP32-term
masses against the exact softmax.
"""

from __future__ import annotations

import itertools
import math

import mpmath
import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle.member import check_member, check_members_ref, split_terms
from pck.member import _host_top_k, member_eps, member_eps32


def vllm_kept(logits: np.ndarray, k: int | None, p: float | None) -> set[int]:
    """vLLM's reference masking (apply_top_k_top_p_pytorch) in NumPy: top-k keeps logits >= the
    k-th largest; top-p sorts ascending and drops tokens whose cumulative mass is <= 1 - p,
    always keeping the largest."""
    lv = logits.astype(np.float64).copy()
    order = np.argsort(lv, kind="stable")
    srt = lv[order]
    if k is not None:
        srt[srt < srt[srt.size - k]] = -np.inf
    if p is not None:
        e = np.exp(srt - np.max(srt))
        cum = np.cumsum(e / e.sum())
        drop = cum <= 1 - p
        drop[-1] = False
        srt[drop] = -np.inf
    return {int(order[i]) for i in range(srt.size) if np.isfinite(srt[i])}


def top_k_sets(logits: np.ndarray, k: int) -> list[set[int]]:
    best = max(sum(logits[list(c)]) for c in itertools.combinations(range(logits.size), k))
    return [
        set(c)
        for c in itertools.combinations(range(logits.size), k)
        if math.isclose(sum(logits[list(c)]), best, rel_tol=0, abs_tol=1e-9)
    ]


small = st.lists(st.integers(-3, 3), min_size=2, max_size=7).map(np.array)


@settings(max_examples=300, deadline=None)
@given(small, st.data())
def test_top_k_count_is_exactly_set_membership(logits: np.ndarray, data: st.DataObject) -> None:
    k = data.draw(st.integers(1, logits.size))
    t = data.draw(st.integers(0, logits.size - 1))
    expected = any(t in s for s in top_k_sets(logits.astype(float), k))
    assert check_member(logits, t, top_k=k).ok == expected


@settings(max_examples=200, deadline=None)
@given(st.lists(st.floats(-6, 6, allow_nan=False), min_size=2, max_size=40).map(np.array), st.data())
def test_every_token_vllm_keeps_is_accepted(logits: np.ndarray, data: st.DataObject) -> None:
    k = data.draw(st.one_of(st.none(), st.integers(1, logits.size)))
    p = data.draw(st.one_of(st.none(), st.floats(0.05, 0.99)))
    for t in vllm_kept(logits, k, p):
        assert check_member(logits, t, top_k=k, top_p=p).ok


def test_rejects_tokens_outside_top_k_or_the_nucleus() -> None:
    logits = np.array([5.0, 4.0, 3.0, 0.0, -1.0])
    assert check_member(logits, 2, top_k=3).ok and not check_member(logits, 3, top_k=3).ok
    v = check_member(logits, 2, top_p=0.5)
    assert not v.ok and v.mass_above > 0.9
    assert check_member(logits, 0, greedy=True).ok and not check_member(logits, 1, greedy=True).ok
    assert not check_member(np.array([1.0, math.nan]), 0).ok
    assert not check_member(logits, 5, top_k=5).ok and not check_member(logits, -1, top_k=1).ok


def test_the_error_bounds_are_tiny_at_llm_vocabularies() -> None:
    assert member_eps(151_936) < 1e-10 and member_eps(2) < 1e-14
    assert member_eps32(151_936) < 1e-6


def test_split_terms_within_bound_of_exact_exponential() -> None:
    """Each FP32 term is within 6 u32 relative (+2^-124) of e^(x - m), checked with mpmath."""
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-140, 0, 4000), rng.uniform(-1, 0, 1000)]).astype(np.float32)
    m = np.float32(0.0)
    mpmath.mp.prec = 120
    terms = split_terms(x, np.full(x.shape, m))
    for xi, ti in zip(x, terms):
        exact = mpmath.e ** (mpmath.mpf(float(xi)) - float(m))
        if float(xi) - float(m) < -128:
            assert ti == 0 or abs(mpmath.mpf(float(ti)) - exact) <= 2.0**-124 + 6 * 2.0**-24 * exact
            continue
        assert abs(mpmath.mpf(float(ti)) - exact) <= 6 * 2.0**-24 * exact + 2.0**-124


def test_host_top_k_limits() -> None:
    assert _host_top_k(None, np.array([5, 20, 500]), 500) == (20, False)
    assert _host_top_k(None, np.array([5, 20, 7]), 500) == (20, True)
    assert _host_top_k(None, np.array([500, 900]), 500) == (0, False)
    assert _host_top_k(None, np.array([0, 3]), 500) == (3, True)  # clipped to >= 1


def _assert_batch_matches_rows(logits, tokens, top_k, top_p, greedy, **kw) -> None:  # type: ignore[no-untyped-def]
    out = check_members_ref(logits, tokens, top_k, top_p, greedy, **kw)
    rows, vocab = logits.shape
    f32 = logits.astype(np.float32)
    for i in range(rows):
        k = None if top_k is None or top_k[i] >= vocab else int(top_k[i])
        p = None if top_p is None or top_p[i] >= 1.0 else float(top_p[i])
        g = bool(greedy[i]) if greedy is not None else False
        ref = check_member(f32[i], int(tokens[i]), k, p, greedy=g)
        assert bool(out["ok"][i]) == ref.ok, i
        if ref.above >= 0:
            assert int(out["above"][i]) == ref.above
        if ref.ok and p is not None and not g:
            assert abs(float(out["mass_above"][i]) - ref.mass_above) <= member_eps32(vocab)


def test_batched_semantics_match_the_reference() -> None:
    """The seeds and mix of the reference's test_the_batched_check_matches_the_reference."""
    rng = np.random.default_rng(0)
    logits = rng.standard_normal((64, 500)) * 3
    logits[:, :5] = 7.0
    tokens = rng.integers(0, 500, 64)
    tokens[:32] = np.argsort(-logits[:32], axis=1)[np.arange(32), rng.integers(0, 20, 32)]
    top_k = rng.choice([1, 5, 20, 500], 64)
    top_p = rng.choice([0.3, 0.9, 1.0], 64)
    greedy = rng.random(64) < 0.1
    _assert_batch_matches_rows(logits.astype(np.float32), tokens, top_k, top_p, greedy)


@pytest.mark.parametrize("host", [False, True])
def test_the_top_k_path_counts_ties_beyond_the_largest_k(host: bool) -> None:
    rng = np.random.default_rng(1)
    rows, vocab = 48, 400
    logits = (rng.standard_normal((rows, vocab)) * 4).astype(np.float32)
    top_k = rng.choice([1, 3, 10, 40], rows)
    for i in range(0, rows, 2):
        order = np.argsort(-logits[i])
        logits[i, order[top_k[i] - 1 : top_k[i] + 29]] = logits[i, order[top_k[i] - 1]]
    tokens = np.array([np.argsort(-row)[rng.integers(0, k)] for row, k in zip(logits, top_k)])
    tokens[::5] = rng.integers(0, vocab, len(tokens[::5]))
    top_p = rng.choice([0.2, 0.6, 0.95], rows)
    out = check_members_ref(logits, tokens, top_k, top_p, top_k_host=top_k if host else None)
    for i in range(rows):
        ref = check_member(logits[i], int(tokens[i]), int(top_k[i]), float(top_p[i]))
        assert bool(out["ok"][i]) == ref.ok, i
        if ref.ok:
            assert abs(float(out["mass_above"][i]) - ref.mass_above) <= member_eps32(vocab)


def test_wide_logits_stay_within_the_bound() -> None:
    rng = np.random.default_rng(2)
    rows, vocab = 16, 5000
    logits = rng.uniform(-300, 40, (rows, vocab)).astype(np.float32)
    logits[:, :50] = rng.uniform(30, 40, (rows, 50)).astype(np.float32)
    tokens = np.argsort(-logits, axis=1)[:, 7]
    out = check_members_ref(logits, tokens, top_p=np.full(rows, 0.99))
    for i in range(rows):
        ref = check_member(logits[i], int(tokens[i]), top_p=0.99)
        assert abs(float(out["mass_above"][i]) - ref.mass_above) <= member_eps32(vocab)


def test_bad_ids_and_a_stale_host_top_k_reject_instead_of_crashing() -> None:
    rng = np.random.default_rng(3)
    logits = rng.standard_normal((4, 50)).astype(np.float32)
    tokens = np.array([-1, 50, 10_000, int(logits[3].argmax())])
    out = check_members_ref(
        logits, tokens, np.array([5, 5, 5, 20]), np.full(4, 0.9), top_k_host=np.array([5, 5, 5, 5])
    )
    assert out["ok"].tolist() == [False, False, False, True]
