"""TEST INFRASTRUCTURE — CPU models of the sampled-token membership check.

`check_member` restates the FP64 per-row reference of `src/pck/member.py:53-81`.
`check_members_ref` restates the batched semantics of `src/pck/member.py:118-197` (the
check vLLM runs per step) in NumPy: exact FP32 comparisons and counts, FP32 softmax terms on
an exact TwoSum split, FP64 sums, the top-(max k) path with ties beyond it, the clamp for a
stale host copy of top-k and the outward-rounded top-p bound.  The HIP kernel must agree with
it exactly on ``ok`` and ``above``, and on ``mass_above`` within `member_eps32` (the FP64
summation order and the last bits of ``expf`` are free within that bound).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
from numpy.typing import NDArray

from pck.fp import next_up
from pck.member import member_eps, member_eps32


@dataclass(frozen=True)
class MemberVerdict:
    ok: bool
    above: int
    mass_above: float


def check_member(
    logits: NDArray[np.floating],
    token: int,
    top_k: int | None = None,
    top_p: float | None = None,
    *,
    greedy: bool = False,
    tol: float = 1e-4,
) -> MemberVerdict:
    """The FP64 reference check of one row (reference `src/pck/member.py:53-81`).

    Reject on NaN or an id outside [0, V); count the logits strictly above the token's;
    reject if that count reaches k (k = 1 for greedy); with top-p, the kept set is the logits
    >= the k-th largest and r = (kept mass strictly above the token) / (kept mass) must stay
    below next_up(p + next_up(tol + member_eps(V))).
    """
    lv = np.asarray(logits, dtype=np.float64)
    if np.isnan(lv).any() or not 0 <= token < lv.size:
        return MemberVerdict(False, -1, math.nan)
    lt = lv[token]
    above = int(np.count_nonzero(lv > lt))
    k = 1 if greedy else top_k
    if k is not None and above >= k:
        return MemberVerdict(False, above, math.nan)
    if greedy or top_p is None or top_p >= 1.0:
        return MemberVerdict(True, above, 0.0)
    kept = np.ones(lv.shape, dtype=bool)
    if top_k is not None and top_k < lv.size:
        kth = np.partition(lv, lv.size - top_k)[lv.size - top_k]
        kept = lv >= kth
    m = lv[kept].max()
    e = np.where(kept, np.exp(lv - m), 0.0)
    r = float(e[lv > lt].sum() / e.sum())
    slack = next_up(tol + member_eps(lv.size))
    return MemberVerdict(bool(r < next_up(top_p + slack)), above, r)


def split_terms(x: NDArray[np.float32], m: NDArray[np.float32]) -> NDArray[np.float32]:
    """FP32 e^(x - m) from the exact split x - m = hi + lo (Knuth's TwoSum), as
    ``expf(hi) + expf(hi) lo``, 0 where hi < -128 or NaN (reference `src/pck/member.py:105-115`)."""
    x = np.asarray(x, dtype=np.float32)
    nm = np.float32(-1) * np.asarray(m, dtype=np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        hi = (x + nm).astype(np.float32)
        bv = (hi - x).astype(np.float32)
        lo = ((x - (hi - bv)) + (nm - bv)).astype(np.float32)
        eh = np.exp(hi).astype(np.float32)
        t = (eh + (eh * lo).astype(np.float32)).astype(np.float32)
    return np.where(hi >= np.float32(-128.0), t, np.float32(0.0)).astype(np.float32)


def check_members_ref(
    logits: NDArray[np.floating],
    tokens: NDArray[np.integer],
    top_k: NDArray[np.integer] | None = None,
    top_p: NDArray[np.floating] | None = None,
    greedy: NDArray[np.bool_] | None = None,
    tol: float = 1e-4,
    top_k_host: NDArray[np.integer] | None = None,
) -> dict[str, NDArray]:
    """Batched membership check with the semantics of `src/pck/member.py:118-197`.

    Returns ``ok`` (B,) bool, ``above`` (B,) int64 and ``mass_above`` (B,) float64.
    """
    lv = np.asarray(logits, dtype=np.float32)
    rows, vocab = lv.shape
    t = np.asarray(tokens).astype(np.int64).reshape(rows)
    in_range = (t >= 0) & (t < vocab)
    lt = lv[np.arange(rows), np.clip(t, 0, vocab - 1)]
    gt = lv > lt[:, None]
    above = gt.sum(1).astype(np.int64)
    finite = ~np.isnan(lv).any(1)
    k = np.full(rows, vocab, dtype=np.int64)
    k_lim, all_k = 0, False
    if top_k is not None:
        k = np.clip(np.asarray(top_k).astype(np.int64), 1, vocab)
        host = top_k_host if top_k_host is not None else np.asarray(top_k)
        hk = np.clip(np.asarray(host).astype(np.int64), 1, vocab)
        lim = hk[hk < vocab]
        k_lim, all_k = (int(lim.max()), lim.size == hk.size) if lim.size else (0, False)
    is_greedy = (
        np.asarray(greedy).astype(bool) if greedy is not None else np.zeros(rows, dtype=bool)
    )
    ok_k = np.where(is_greedy, 1, k)
    ok = finite & in_range & (above < ok_k)
    mass_above = np.zeros(rows)
    if top_p is not None:
        p = np.asarray(top_p).astype(np.float64)
        r = np.empty(rows)
        desc = -np.sort(-lv, axis=1, kind="stable") if k_lim else None
        for i in range(rows):
            row = lv[i]
            if all_k or (k_lim and k[i] < vocab):
                kth = desc[i, min(k[i], k_lim) - 1]
                kept = row >= kth
            else:
                kept = np.ones(vocab, dtype=bool)
            m = row[kept].max() if kept.any() else np.float32(-np.inf)
            e = np.where(kept, split_terms(row, m), np.float32(0.0)).astype(np.float64)
            z = e.sum()
            a = e[gt[i] & kept].sum()
            with np.errstate(invalid="ignore", divide="ignore"):
                r[i] = a / z
        mass_above = np.where(p < 1.0, r, 0.0)
        slack = next_up(tol + member_eps32(vocab))
        high = np.nextafter(p + slack, np.inf)
        with np.errstate(invalid="ignore"):
            topp_ok = (p >= 1.0) | is_greedy | (r < high)
        ok = ok & topp_ok
    return {"ok": ok, "above": above, "mass_above": mass_above}
