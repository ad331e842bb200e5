"""The HIP membership kernel against the oracle: ``ok`` and ``above`` exactly equal to the
batched reference semantics (oracle.member.check_members_ref) and to the per-row FP64
reference; ``mass_above`` within member_eps32 of the FP64 reference.  Covers the reference's
tests/test_member.py batched cases, the LDS fast path and both fallbacks (candidate overflow,
k above 1024), and the BASELINE workload (256 x 151,936 logits, top-k 50, top-p 0.9) with 1% of
tokens replaced by out-of-set tokens that must all be flagged, with no false alarm."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.member import check_member, check_members_ref
from pck.member import check_members, member_eps32

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def run(logits, tokens, top_k=None, top_p=None, greedy=None, top_k_host=None, tol=1e-4):  # type: ignore[no-untyped-def]
    t = lambda a, dt=None: None if a is None else torch.as_tensor(a, dtype=dt).cuda()  # noqa: E731
    out = check_members(
        t(logits, torch.float32), t(tokens), t(top_k), t(top_p), t(greedy), tol, top_k_host
    )
    return {k: v.cpu().numpy() for k, v in out.items()}


def assert_matches_oracle(logits, tokens, top_k=None, top_p=None, greedy=None, top_k_host=None) -> None:  # type: ignore[no-untyped-def]
    got = run(logits, tokens, top_k, top_p, greedy, top_k_host)
    want = check_members_ref(logits, tokens, top_k, top_p, greedy, top_k_host=top_k_host)
    np.testing.assert_array_equal(got["ok"], want["ok"])
    np.testing.assert_array_equal(got["above"], want["above"])
    vocab = logits.shape[1]
    if top_p is not None:
        finite = np.isfinite(want["mass_above"])
        assert np.all(np.abs(got["mass_above"][finite] - want["mass_above"][finite]) <= 2 * member_eps32(vocab))


def test_the_batched_check_matches_the_reference() -> None:
    rng = np.random.default_rng(0)
    logits = (rng.standard_normal((64, 500)) * 3).astype(np.float32)
    logits[:, :5] = 7.0
    tokens = rng.integers(0, 500, 64)
    tokens[:32] = np.argsort(-logits[:32], axis=1)[np.arange(32), rng.integers(0, 20, 32)]
    top_k = rng.choice([1, 5, 20, 500], 64)
    top_p = rng.choice([0.3, 0.9, 1.0], 64)
    greedy = rng.random(64) < 0.1
    out = run(logits, tokens, top_k, top_p, greedy)
    for i in range(64):
        k = None if top_k[i] == 500 else int(top_k[i])
        p = None if top_p[i] == 1.0 else float(top_p[i])
        ref = check_member(logits[i], int(tokens[i]), k, p, greedy=bool(greedy[i]))
        assert bool(out["ok"][i]) == ref.ok, i
        assert int(out["above"][i]) == ref.above
        if ref.ok and p is not None and not greedy[i]:
            assert abs(float(out["mass_above"][i]) - ref.mass_above) <= member_eps32(500)
    assert_matches_oracle(logits, tokens, top_k, top_p, greedy)


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
    out = run(logits, tokens, top_k.astype(np.int32), top_p, top_k_host=top_k if host else None)
    for i in range(rows):
        ref = check_member(logits[i], int(tokens[i]), int(top_k[i]), float(top_p[i]))
        assert bool(out["ok"][i]) == ref.ok, i
        if ref.ok:
            assert abs(float(out["mass_above"][i]) - ref.mass_above) <= member_eps32(vocab)


def test_fp32_terms_stay_within_the_bound_on_wide_logits() -> None:
    rng = np.random.default_rng(2)
    rows, vocab = 16, 5000
    logits = rng.uniform(-300, 40, (rows, vocab)).astype(np.float32)
    logits[:, :50] = rng.uniform(30, 40, (rows, 50)).astype(np.float32)
    tokens = np.argsort(-logits, axis=1)[:, 7]
    out = run(logits, tokens, top_p=np.full(rows, 0.99))
    for i in range(rows):
        ref = check_member(logits[i], int(tokens[i]), top_p=0.99)
        assert abs(float(out["mass_above"][i]) - ref.mass_above) <= member_eps32(vocab)


def test_bad_token_ids_and_a_stale_host_top_k_reject_instead_of_crashing() -> None:
    rng = np.random.default_rng(3)
    logits = rng.standard_normal((4, 50)).astype(np.float32)
    tokens = np.array([-1, 50, 10_000, int(logits[3].argmax())])
    out = run(logits, tokens, np.array([5, 5, 5, 20], dtype=np.int32), np.full(4, 0.9),
              top_k_host=np.array([5, 5, 5, 5]))  # fmt: skip
    assert out["ok"].tolist() == [False, False, False, True]


def test_nan_rows_reject() -> None:
    logits = np.random.default_rng(4).standard_normal((3, 300)).astype(np.float32)
    logits[1, 17] = np.nan
    out = run(logits, np.array([0, 0, 0]), top_p=np.full(3, 0.999999))
    assert not out["ok"][1] and out["ok"][0] == check_member(logits[0], 0, top_p=0.999999).ok


CASES = ["all_equal", "many_ties", "k_above_1024", "keep_all_rows", "mixed", "k_700",
         "k_700_offset", "one_wave_overflows", "wide_window"]  # fmt: skip


@pytest.mark.parametrize("case", CASES)
def test_fallback_paths_match_the_oracle(case: str) -> None:
    """Rows whose candidate set overflows LDS, k_eff above 1024, rows without top-k.  k_700 and
    k_700_offset leave ~1400 candidates (several per lane of each wave's segment, none
    overflowing), spread over four binades or packed into one.  one_wave_overflows puts 512
    equal maxima in the stream slots of one wave only (that wave's segment overflows while the
    row's total fits).  wide_window plants three huge logits per row among ordinary candidates
    (rows with top-k 50 hold at most one candidate per lane, rows with 700 several)."""
    rng = np.random.default_rng(5)
    rows, vocab = 8, 20000
    if case == "one_wave_overflows":
        rows, vocab = 2, 151_936
    logits = (rng.standard_normal((rows, vocab)) * 2).astype(np.float32)
    top_k = np.full(rows, 50)
    if case in ("k_700", "k_700_offset"):
        top_k[:] = 700
        if case == "k_700_offset":
            logits += 100.0
    elif case == "wide_window":
        for r in range(rows):
            logits[r, rng.choice(vocab, 3, replace=False)] = [1e20, 3e10, 7e5]
        top_k[rows // 2 :] = 700
    elif case == "one_wave_overflows":
        # the stream starts at logit 16384; lane t of the workgroup reads quad 4096 + t +
        # 1024 j, so wave 3 (lanes 192..255) reads logits 16384 + 4096 j + 768 .. + 1023
        for j in range(2):
            start = 16384 + 4096 * j + 768
            logits[:, start : start + 256] = 50.0
    elif case == "all_equal":
        logits[:] = 1.25
    elif case == "many_ties":
        logits[:, : vocab // 2] = 3.0  # 10000 values tied at the top
    elif case == "k_above_1024":
        top_k[:] = 3000
    elif case == "keep_all_rows":
        top_k[::2] = vocab
    else:
        top_k = rng.choice([1, 50, 2000, vocab], rows)
        logits[0] = 0.5
    tokens = np.argsort(-logits, axis=1, kind="stable")[np.arange(rows), rng.integers(0, 40, rows)]
    tokens[1] = int(np.argmin(logits[1]))
    top_p = np.full(rows, 0.9)
    assert_matches_oracle(logits, tokens, top_k, top_p)
    assert_matches_oracle(logits, tokens, top_k, top_p, top_k_host=top_k)


@pytest.mark.parametrize("vocab", [20001, 20003, 151937])
def test_odd_vocab_rows_take_every_alignment(vocab: int) -> None:
    """With an odd vocab the rows start at every 4-byte offset: aligned rows end in an
    element tail, the others stream element by element with lanes dropping out at the end of
    each range (the per-wave candidate counts must survive both), and short prefixes are
    re-read from memory.  Top-k + top-p rows (the candidate path) and rows without a top-k."""
    rng = np.random.default_rng(vocab)
    rows = 8
    logits = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    hot = rng.integers(0, vocab, (rows, 6))
    logits[np.arange(rows)[:, None], hot] += 12.0
    top_k = np.array([50, 50, 50, 50, 200, 700, vocab, 50])
    order = np.argsort(-logits, axis=1, kind="stable")
    tokens = order[np.arange(rows), rng.integers(0, 60, rows)]
    top_p = np.full(rows, 0.9)
    assert_matches_oracle(logits, tokens, top_k, top_p)
    assert_matches_oracle(logits, tokens, top_k, top_p, top_k_host=top_k)


def vllm_kept_row(row: np.ndarray, k: int, p: float) -> np.ndarray:
    """Token ids vLLM's own top-k then top-p masking keeps (apply_top_k_top_p_pytorch)."""
    order = np.argsort(row.astype(np.float64), kind="stable")
    srt = row.astype(np.float64)[order]
    srt[srt < srt[srt.size - k]] = -np.inf
    e = np.exp(srt - srt.max())
    cum = np.cumsum(e / e.sum())
    drop = cum <= 1 - p
    drop[-1] = False
    return order[np.isfinite(srt) & ~drop]


def test_baseline_workload_flags_every_planted_token() -> None:
    """256 x 151,936 FP32 logits ~ N(0, 3) with 8 hot tokens per row at +10..+20, top-k 50,
    top-p 0.9, T = 1: honest tokens drawn from vLLM's kept set all pass; 1% of rows get an
    out-of-set token (the row's argmin, as the plugin's fault injection does, or a token with at
    least 50 larger logits) and every one is flagged."""
    rows, vocab = 256, 151_936
    rng = np.random.default_rng(0)
    logits = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    for i in range(rows):
        hot = rng.choice(vocab, 8, replace=False)
        logits[i, hot] += rng.uniform(10, 20, 8).astype(np.float32)
    tokens = np.array([rng.choice(vllm_kept_row(logits[i], 50, 0.9)) for i in range(rows)])
    bad = rng.choice(rows, rows // 100, replace=False)
    for j, i in enumerate(bad):
        order = np.argsort(-logits[i])
        tokens[i] = int(np.argmin(logits[i])) if j % 2 == 0 else int(order[rng.integers(60, 5000)])
    top_k = np.full(rows, 50)
    top_p = np.full(rows, 0.9)
    out = run(logits, tokens, top_k, top_p, top_k_host=top_k)
    planted = np.zeros(rows, dtype=bool)
    planted[bad] = True
    assert not out["ok"][planted].any()  # every planted token caught
    assert out["ok"][~planted].all()  # no false alarm
    want = check_members_ref(logits[:32], tokens[:32], top_k[:32], top_p[:32], top_k_host=top_k[:32])
    np.testing.assert_array_equal(out["ok"][:32], want["ok"])
    np.testing.assert_array_equal(out["above"][:32], want["above"])
    for i in range(8):
        ref = check_member(logits[i], int(tokens[i]), 50, 0.9)
        if ref.ok:
            assert abs(float(out["mass_above"][i]) - ref.mass_above) <= member_eps32(vocab)


def test_top_k_outside_one_to_vocab_is_clamped_like_the_reference() -> None:
    """Requested top-k values below 1 or above V act as 1 and V (reference
    src/pck/member.py:153); the kernel clamps them, so no host-side clamp launch is needed."""
    rng = np.random.default_rng(3)
    logits = (rng.standard_normal((6, 300)) * 3).astype(np.float32)
    order = np.argsort(-logits, axis=1)
    tokens = order[np.arange(6), [0, 1, 0, 5, 2, 299]]
    top_k = np.array([0, -3, 1, 10**9, 301, 300])
    clamped = np.clip(top_k, 1, 300)
    got = run(logits, tokens, top_k, np.full(6, 0.9), top_k_host=clamped)
    want = run(logits, tokens, clamped, np.full(6, 0.9), top_k_host=clamped)
    for key in ("ok", "above"):
        np.testing.assert_array_equal(got[key], want[key])
    # candidates meet in LDS in arrival order, so the FP64 sums may differ in their last bits
    assert np.all(np.abs(got["mass_above"] - want["mass_above"]) <= 2 * member_eps32(300))
    assert_matches_oracle(logits, tokens, clamped, np.full(6, 0.9), top_k_host=clamped)


def test_request_index_outside_the_temperature_array_rejects_the_row() -> None:
    """The sampler-hook entry reads greedy through a per-row request index: an index outside
    [0, len(temperature)) rejects that row (counted as rejected in the device totals) without
    reading past the array, and the other rows keep their verdicts."""
    from pck.member import launch_check, new_totals

    rng = np.random.default_rng(11)
    rows, vocab = 8, 3000
    logits = torch.from_numpy(rng.standard_normal((rows, vocab)).astype(np.float32)).cuda()
    tokens = logits.argmax(dim=1)  # allowed under any top-k / top-p: every row passes
    temperature = torch.tensor([0.0, 1.0, 0.7], device="cuda")
    good = torch.tensor([0, 1, 2, 1, 0, 2, 1, 0], device="cuda")
    ref = launch_check(logits, tokens, temperature=temperature, temperature_index=good)
    assert bool(ref["ok"].all())
    bad = good.clone()
    bad[2], bad[5] = 3, -1  # past the end, negative
    totals = new_totals(logits.device)
    out = launch_check(logits, tokens, temperature=temperature, temperature_index=bad, totals=totals)
    assert out["ok"].tolist() == [True, True, False, True, True, False, True, True]
    assert int(totals[0]) == rows and int(totals[1]) == 2
