"""Membership checks for samplers that return a token, not a set (reference `src/pck/member.py`).

For a row of logits ``l``, the sampled token ``t`` and the request's ``top_k`` / ``top_p``
(vLLM's order: top-k first, then top-p over the survivors):

  top-k   accept iff fewer than ``k`` logits are strictly larger than ``l[t]``;
  top-p   K = logits >= the k-th largest (all without top-k); r = share of K's softmax mass
          strictly above ``t``; accept iff r < next_up(p + slack), slack = tol + eps;
  greedy  accept iff no logit is strictly larger than ``l[t]``;
  NaN logits or an id outside [0, V) reject.

`check_members` runs the whole batch in one launch of the HIP kernel (`pck_check_members_ex`:
exact FP32 comparisons, FP32 softmax terms on an exact split argument, FP64 sums); it needs the
logits on the GPU, and `launch_check` also keeps running totals on the device.  `check_member`
is the reference's FP64 check of one row on the CPU.  `member_eps` / `member_eps32` are the
error bounds the slack is built from (reference `src/pck/member.py:37-41,84-102`).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any

import numpy as np

from pck.fp import U32, U64, gamma, next_up, softmax_eps


def member_eps(vocab: int) -> float:
    """Error bound of the FP64 reference check: `pck.fp.softmax_eps` with the logits used
    directly (reference `src/pck/member.py:37-41`)."""
    return softmax_eps(vocab)


@dataclass(frozen=True)
class MemberVerdict:
    """The verdict of `check_member` (reference `src/pck/member.py:45-50`)."""

    ok: bool
    above: int
    """Logits strictly larger than the sampled token's (-1 for NaN logits or a bad id)."""
    mass_above: float
    """Fraction of the kept softmax mass strictly above the token (0 without top-p)."""


def check_member(
    logits: Any,
    token: int,
    top_k: int | None = None,
    top_p: float | None = None,
    *,
    greedy: bool = False,
    tol: float = 1e-4,
) -> MemberVerdict:
    """One row, in FP64 on the CPU (reference `src/pck/member.py:53-81`): NaN logits or an id
    outside [0, V) reject; so does a token with k or more larger logits (k = 1 when greedy);
    with top-p below 1 the kept set is every logit >= the k-th largest (all without top-k), r
    is its softmax mass strictly above the token, and the row passes iff
    r < next_up(top_p + next_up(tol + member_eps(V)))."""
    row = np.asarray(logits, dtype=np.float64)
    if np.isnan(row).any() or not 0 <= token < row.size:
        return MemberVerdict(False, -1, math.nan)
    lt = row[token]
    above = int(np.count_nonzero(row > lt))
    limit = 1 if greedy else top_k
    if limit is not None and above >= limit:
        return MemberVerdict(False, above, math.nan)
    if greedy or top_p is None or top_p >= 1.0:
        return MemberVerdict(True, above, 0.0)
    kept = np.ones(row.size, dtype=bool)
    if top_k is not None and top_k < row.size:
        kept = row >= np.sort(row)[row.size - top_k]  # the k-th largest
    terms = np.where(kept, np.exp(row - row[kept].max()), 0.0)
    r = float(terms[row > lt].sum() / terms.sum())
    slack = next_up(tol + member_eps(row.size))
    return MemberVerdict(bool(r < next_up(top_p + slack)), above, r)


def member_eps32(vocab: int) -> float:
    """Error bound of r for FP32 split-argument terms summed in FP64 (reference
    `src/pck/member.py:84-102`): each term within 6 u32 relative plus 2^-124 absolute (a
    2-ulp ``expf``, two roundings, terms below e^-128 dropped), both sums within
    gamma_{V+2}(u64), so E = 6 u32 + V 2^-124 + gamma_{V+2}(u64) (1 + 6 u32 + V 2^-124) and
    the quotient is within 2E / (1 - E) + u64."""
    tiny = math.ldexp(vocab, -124)
    e = 6 * U32 + tiny + gamma(vocab + 2, U64) * (1 + 6 * U32 + tiny)
    return 2 * e / (1 - e) + U64


def _host_top_k(top_k: Any, top_k_host: Any, vocab: int) -> tuple[int, bool]:
    """(k_lim, all_k) from the host copy of top-k (reference `src/pck/member.py:152-157`):
    the largest top-k below the vocabulary and whether every row has one."""
    host = top_k_host if top_k_host is not None else top_k.cpu().numpy()
    hk = np.clip(np.asarray(host).astype(np.int64), 1, vocab)
    lim = hk[hk < vocab]
    return (int(lim.max()), lim.size == hk.size) if lim.size else (0, False)


EXCESS_NONE = -1.0
"""max_excess before any accepted top-p row (r - p >= -1 always)."""


def excess_key(v: float) -> int:
    """The order-preserving 64-bit key the membership kernel keeps the running maximum of
    r - p in (a larger value has a larger key)."""
    u = int(np.array([v], dtype=np.float64).view(np.uint64)[0])
    return (~u & (2**64 - 1)) if u >> 63 else u | (1 << 63)


def excess_value(key: int) -> float:
    """Inverse of `excess_key`."""
    u = (key & ~(1 << 63)) if key >> 63 else (~key & (2**64 - 1))
    return float(np.array([u], dtype=np.uint64).view(np.float64)[0])


def key_as_int64(key: int) -> int:
    """The signed 64-bit integer with the same bits as the unsigned ``key``."""
    return key - 2**64 if key >= 2**63 else key


def new_totals(device: Any) -> Any:
    """A device buffer for `launch_check` to add a batch's counts into: rows, rejected,
    injected, caught, false alarms, and the key of the largest r - p so far (none yet)."""
    import torch

    host = torch.zeros(6, dtype=torch.int64)
    host[5] = key_as_int64(excess_key(EXCESS_NONE))
    return host.to(device)


def launch_check(
    logits: Any,
    tokens: Any,
    top_k: Any = None,
    top_p: Any = None,
    greedy: Any = None,
    tol: float = 1e-4,
    top_k_host: Any = None,
    *,
    temperature: Any = None,
    temperature_index: Any = None,
    injected: Any = None,
    totals: Any = None,
    outputs: bool = True,
) -> dict[str, Any] | None:
    """One launch of the membership kernel (`pck_check_members_ex`) over a batch.

    Beside `check_members`'s arguments: ``temperature`` (requests,) FP32 with
    ``temperature_index`` (B,) makes row r greedy iff temperature[index[r]] == 0 (instead of
    ``greedy``), and rejects a row whose index is outside [0, requests); ``top_p`` may be FP32 (read as is) or FP64; ``injected`` (B,) bool marks planted
    faults; ``totals`` (from `new_totals`) receives the batch's counts on the device.  Returns
    the outputs (``ok``, ``above``, ``mass_above``) unless ``outputs`` is False.  Never
    synchronises: top-k's host copy is ``top_k_host`` (or one copy of ``top_k``)."""
    import torch

    from pck.cuda._lib import PckMemberArgs, check, lib, stream_handle

    if not logits.is_cuda:
        raise RuntimeError(
            "check_members runs the HIP membership kernel and needs logits on the GPU, "
            f"got {logits.device}"
        )
    device = logits.device
    lv = logits.float().contiguous()
    if lv.dim() != 2:
        raise RuntimeError(f"expected logits of shape (B, V), got {list(lv.shape)}")
    rows, vocab = lv.shape
    keep = [lv]

    def dev(x: Any, dtype: Any, name: str) -> int | None:
        if x is None:
            return None
        t = x.to(device=device, dtype=dtype).reshape(rows).contiguous() if dtype else x
        if t.numel() != rows:
            raise RuntimeError(f"{name} must have {rows} entries, got {t.numel()}")
        keep.append(t)
        return int(t.data_ptr())

    a = PckMemberArgs()
    a.logits, a.rows, a.vocab = lv.data_ptr(), rows, vocab
    a.tokens = dev(tokens, torch.long, "tokens")
    if top_k is not None:  # clamped to [1, V] by the kernel
        a.top_k = dev(top_k, torch.long, "top_k")
        a.k_lim, a.all_k = _host_top_k(top_k, top_k_host, vocab)
    if top_p is not None:
        fp32 = top_p.dtype == torch.float32
        a.top_p = dev(top_p, torch.float32 if fp32 else torch.float64, "top_p")
        a.top_p_fp32 = int(fp32)
    if temperature is not None:
        t = temperature.to(device=device, dtype=torch.float32).contiguous()
        keep.append(t)
        a.temperature = t.data_ptr()
        a.temperature_count = t.numel()
        a.temperature_index = dev(temperature_index, torch.long, "temperature_index")
    elif greedy is not None:  # a bool tensor is read as its bytes (0 or 1)
        g = greedy.to(device=device, dtype=torch.bool).reshape(rows).contiguous().view(torch.uint8)
        a.greedy = dev(g, None, "greedy")
    if injected is not None:
        inj = injected.to(device=device, dtype=torch.bool).reshape(rows).contiguous().view(torch.uint8)
        a.injected = dev(inj, None, "injected")
    if totals is not None:
        if not (totals.is_cuda and totals.device == device and totals.dtype == torch.int64
                and totals.numel() == 6 and totals.is_contiguous()):  # fmt: skip
            raise RuntimeError("totals must be a contiguous (6,) int64 tensor on the logits' device")
        a.totals = totals.data_ptr()
    out = None
    if outputs:
        # the three outputs in one allocation: [mass_above | above | ok]
        buf = torch.empty(17 * rows, dtype=torch.uint8, device=device)
        out = {
            "ok": buf[16 * rows :].view(torch.bool),
            "above": buf[8 * rows : 16 * rows].view(torch.int64),
            "mass_above": buf[: 8 * rows].view(torch.float64),
        }
        a.ok, a.above, a.mass_above = (
            out["ok"].data_ptr(), out["above"].data_ptr(), out["mass_above"].data_ptr()
        )  # fmt: skip
    if rows == 0:
        return out
    a.slack = next_up(tol + member_eps32(vocab))
    with torch.cuda.device(device):
        err = lib().pck_check_members_ex(a, stream_handle(device))
    check(err, "membership check launch")
    return out


def check_members(
    logits: Any,
    tokens: Any,
    top_k: Any = None,
    top_p: Any = None,
    greedy: Any = None,
    tol: float = 1e-4,
    top_k_host: Any = None,
) -> dict[str, Any]:
    """The membership check for a batch (reference `src/pck/member.py:118-197`).

    ``logits`` (B, V) on the GPU (FP32, or FP16 / BF16, widened exactly); ``tokens`` (B,);
    optional per-row ``top_k`` (B,) ints (V = no top-k), ``top_p`` (B,) floats (1 = none) and
    ``greedy`` (B,) bools.  ``top_k_host`` is the same top-k values on the host (any array with
    the same set of values); with it the check never synchronises the device, without it they
    are copied from ``top_k`` once.  Returns device tensors ``ok`` (B,) bool, ``above`` (B,)
    int64 and ``mass_above`` (B,) float64.
    """
    out = launch_check(logits, tokens, top_k, top_p, greedy, tol, top_k_host)
    assert out is not None
    return out
