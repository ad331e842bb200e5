"""Membership checks for samplers that return a token, not a set (reference `src/pck/member.py`).

For a row of logits ``l``, the sampled token ``t`` and the request's ``top_k`` / ``top_p``
(vLLM's order: top-k first, then top-p over the survivors):

  top-k   accept iff fewer than ``k`` logits are strictly larger than ``l[t]``;
  top-p   K = logits >= the k-th largest (all without top-k); r = share of K's softmax mass
          strictly above ``t``; accept iff r < next_up(p + slack), slack = tol + eps;
  greedy  accept iff no logit is strictly larger than ``l[t]``;
  NaN logits or an id outside [0, V) reject.

`check_members` runs the whole batch in one launch of the HIP kernel `pck_check_members`
(exact FP32 comparisons, FP32 softmax terms on an exact split argument, FP64 sums); it needs
the logits on the GPU.  `member_eps` / `member_eps32` are the error bounds the slack is built
from (reference `src/pck/member.py:37-41,84-102`).
"""

from __future__ import annotations

import math
from typing import Any

import numpy as np

from pck.fp import U32, U64, gamma, next_up, softmax_eps


def member_eps(vocab: int) -> float:
    """Error bound of the FP64 reference check: `pck.fp.softmax_eps` with the logits used
    directly (reference `src/pck/member.py:37-41`)."""
    return softmax_eps(vocab)


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
    import torch

    from pck.cuda._lib import check, lib, stream_handle

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
    t = tokens.reshape(rows).to(device=device, dtype=torch.long).contiguous()
    k_dev = None
    k_lim, all_k = 0, False
    if top_k is not None:  # clamped to [1, V] by the kernel
        k_dev = top_k.to(device=device, dtype=torch.long).reshape(rows).contiguous()
        k_lim, all_k = _host_top_k(top_k, top_k_host, vocab)
    p_dev = None
    if top_p is not None:
        p_dev = top_p.to(device=device, dtype=torch.float64).reshape(rows).contiguous()
    g_dev = None
    if greedy is not None:  # a bool tensor is read as its bytes (0 or 1)
        g_dev = greedy.to(device=device, dtype=torch.bool).reshape(rows).contiguous().view(torch.uint8)
    # the three outputs in one allocation: [mass_above | above | ok]
    out = torch.empty(17 * rows, dtype=torch.uint8, device=device)
    mass_above = out[: 8 * rows].view(torch.float64)
    above = out[8 * rows : 16 * rows].view(torch.int64)
    ok = out[16 * rows :].view(torch.bool)
    if rows == 0:
        return {"ok": ok, "above": above, "mass_above": mass_above}
    slack = next_up(tol + member_eps32(vocab))

    def ptr(x: Any) -> int | None:
        return None if x is None else x.data_ptr()

    with torch.cuda.device(device):
        err = lib().pck_check_members(
            lv.data_ptr(), rows, vocab, t.data_ptr(), ptr(k_dev), ptr(p_dev), ptr(g_dev), slack,
            k_lim, int(all_k), ok.data_ptr(), above.data_ptr(), mass_above.data_ptr(),
            stream_handle(device),
        )  # fmt: skip
    check(err, "membership check launch")
    return {"ok": ok, "above": above, "mass_above": mass_above}
