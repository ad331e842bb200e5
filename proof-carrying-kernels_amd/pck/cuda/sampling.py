"""Trusted top-k / top-p set checker on the GPU, and untrusted GPU samplers to test it
(reference `src/pck/cuda/sampling.py`).

``check_topk_gpu`` and ``check_topp_gpu`` run the library's set checker (`pck_sampling_check`):
exact FP32 comparisons for the top-k prefix property, FP64 masses for top-p minimality, one
call for a batch of rows.  Selections are ``(B, L)`` int64 tensors with per-row lengths, so
top-p nuclei of different sizes share one call.  ``topk_sample``, ``topp_select`` and
``sharded_topk_gpu`` are the code under test, built from torch operations; they are not
trusted.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from pck.cuda._lib import check, lib, stream_handle
from pck.cuda.checker import _check_tensor
from pck.fp import U32, U64, ceil_div, gamma

BLOCKS_PER_SM = 4  # workgroups per CU the default segment count aims for
MIN_SEGMENT = 4096  # logits per segment, at least


@dataclass(frozen=True)
class SamplingCheck:
    """Per-row checker outputs, each of shape (B,) (reference `cuda/sampling.py:26-34`)."""

    passed: torch.Tensor
    min_selected: torch.Tensor
    max_rejected: torch.Tensor
    mass: torch.Tensor
    mass_without_smallest: torch.Tensor


def default_segments(logits: torch.Tensor) -> int:
    """Split each row so that the grid has about ``BLOCKS_PER_SM`` workgroups per CU, with at
    least ``MIN_SEGMENT`` logits per segment (reference `cuda/sampling.py:43-47`)."""
    rows, vocab = logits.shape
    cus = torch.cuda.get_device_properties(logits.device).multi_processor_count
    return max(1, min(ceil_div(BLOCKS_PER_SM * cus, rows), ceil_div(vocab, MIN_SEGMENT)))


def sampling_check(
    logits: torch.Tensor, selected: torch.Tensor, lengths: torch.Tensor | None, k: int,
    top_p: bool, p: float, temperature: float, slack: float, segments: int,
) -> list[torch.Tensor]:  # fmt: skip
    """The pybind ``sampling_check`` of the reference (`bindings.cpp:260-298`): the same
    validation, in the same order and with the same messages; returns
    [passed, min_selected, max_rejected, mass, mass_without_smallest], enqueued on the
    current stream.  ``lengths`` None means every row's selection is its whole width (the
    reference's top-k call passes a tensor filled with k; here no such tensor is built)."""
    if not logits.is_cuda:
        raise RuntimeError("logits must be a CUDA tensor")
    device = logits.device
    _check_tensor(logits, "logits", torch.float32, device)
    _check_tensor(selected, "selected", torch.int64, device)
    if lengths is not None:
        _check_tensor(lengths, "lengths", torch.int64, device)
    if not (logits.dim() == 2 and selected.dim() == 2 and (lengths is None or lengths.dim() == 1)):
        raise RuntimeError("expected logits (B, V), selected (B, L), lengths (B,)")
    rows, vocab = logits.shape
    max_len = selected.size(1)
    if not (selected.size(0) == rows and (lengths is None or lengths.size(0) == rows)):
        raise RuntimeError("batch sizes differ")
    if not (rows >= 1 and vocab >= 1 and max_len >= 1):
        raise RuntimeError("empty input")
    if rows > 65535:
        raise RuntimeError("too many rows")
    if not (1 <= segments <= vocab and segments <= 2**31 - 1):
        raise RuntimeError(f"segments must be in [1, V], got {segments}")
    if not (temperature > 0 and slack >= 0):
        raise RuntimeError("temperature must be positive, slack >= 0")
    handle = lib()
    # short selections are read per segment into LDS; longer ones need the zeroed bitmap
    if handle.pck_sampling_needs_scratch(vocab, max_len, segments):
        scratch = torch.zeros((rows, handle.pck_sampling_scratch_words(vocab)), dtype=torch.int32, device=device)
        scratch_ptr = scratch.data_ptr()
    else:
        scratch_ptr = 0
    # one allocation for the partials and the five outputs, each at an offset aligned for its
    # type: [partials | mass | without | min_selected | max_rejected | passed]
    part = rows * segments * handle.pck_sampling_partial_bytes()  # a multiple of 8
    buf = torch.empty(part + 25 * rows, dtype=torch.uint8, device=device)
    partials = buf[:part]
    mass = buf[part : part + 8 * rows].view(torch.float64)
    without = buf[part + 8 * rows : part + 16 * rows].view(torch.float64)
    min_sel = buf[part + 16 * rows : part + 20 * rows].view(torch.float32)
    max_rej = buf[part + 20 * rows : part + 24 * rows].view(torch.float32)
    passed = buf[part + 24 * rows : part + 25 * rows].view(torch.bool)
    with torch.cuda.device(device):
        err = handle.pck_sampling_check(
            logits.data_ptr(), selected.data_ptr(), None if lengths is None else lengths.data_ptr(),
            rows, vocab, max_len, k,
            int(top_p), p, temperature, slack, segments, scratch_ptr, partials.data_ptr(),
            passed.data_ptr(), min_sel.data_ptr(), max_rej.data_ptr(), mass.data_ptr(),
            without.data_ptr(), stream_handle(device),
        )  # fmt: skip
    check(err, "sampling checker launch")
    return [passed, min_sel, max_rej, mass, without]


def check_topk_gpu(
    logits: torch.Tensor, selected: torch.Tensor, k: int, segments: int | None = None
) -> SamplingCheck:
    """Check that each row of ``selected`` (B, k) is a valid top-k set of ``logits`` (B, V)
    (reference `cuda/sampling.py:50-58`)."""
    segs = default_segments(logits) if segments is None else segments
    out = sampling_check(logits, selected, None, k, False, 1.0, 1.0, 0.0, segs)
    return SamplingCheck(*out)


def topp_slack(vocab: int, segments: int, tol: float) -> float:
    """The sampler's ``tol`` plus this checker's own rounding (reference
    `cuda/sampling.py:71-88`): each term is FP32 expf on a split argument (within 2 ulp, plus
    under 2 u32 for the split and the FMA: 6 u32 relative) or below 2^-148 where dropped;
    each of the S segment partials is rescaled with one FP64 exp, multiply and add; the
    largest term is exactly 1.  Each mass is then within 16 u32 + V 2^-146 +
    gamma_{V + 3S + 16}(u64), rounded up."""
    own = 16 * U32 + math.ldexp(vocab, -146) + gamma(vocab + 3 * segments + 16, U64)
    return math.nextafter(tol + own, math.inf)


def check_topp_gpu(
    logits: torch.Tensor,
    selected: torch.Tensor,
    lengths: torch.Tensor,
    p: float,
    temperature: float = 1.0,
    tol: float = 1e-6,
    segments: int | None = None,
) -> SamplingCheck:
    """Check that ``selected[b, :lengths[b]]`` is a valid, minimal top-p nucleus of row b
    (reference `cuda/sampling.py:61-93`).  ``tol`` is the sampler's declared probability error;
    the checker adds its own rounding slack (`topp_slack`)."""
    if not 0 < p <= 1:
        raise ValueError(f"p must be in (0, 1], got {p}")
    if tol < 0:
        raise ValueError(f"tol must be non-negative, got {tol}")
    segs = default_segments(logits) if segments is None else segments
    slack = topp_slack(logits.shape[1], segs, tol)
    out = sampling_check(logits, selected, lengths, 0, True, p, temperature, slack, segs)
    return SamplingCheck(*out)


def topk_sample(
    logits: torch.Tensor, k: int, generator: torch.Generator | None = None
) -> tuple[torch.Tensor, torch.Tensor]:
    """Untrusted top-k sampler for the checker to judge (the role of the reference's
    `cuda/sampling.py:96-103`): the k largest logits per row, then one token drawn from their
    softmax by the Gumbel-max trick (argmax of value + Gumbel noise).  Returns (selected (B, k),
    token (B,))."""
    values, idx = torch.topk(logits, k, dim=-1)
    u = torch.rand(values.shape, generator=generator, device=logits.device, dtype=torch.float64)
    gumbel = -torch.log(-torch.log(u.clamp_min(1e-300)))
    pick = (values.double() + gumbel).argmax(dim=-1, keepdim=True)
    return idx, idx.gather(-1, pick).squeeze(-1)


def topp_select(
    logits: torch.Tensor, p: float, temperature: float = 1.0
) -> tuple[torch.Tensor, torch.Tensor]:
    """Untrusted top-p selection for the checker to judge (the role of the reference's
    `cuda/sampling.py:106-121`): logits sorted in descending order (stable, so ties keep
    index order), their probabilities exp((l - max) / T) normalised in FP64, and the shortest
    prefix whose cumulative mass reaches p (searchsorted).  Returns (selected (B, V) indices in
    that order, lengths (B,)); the first lengths[b] entries of row b are the nucleus."""
    scaled = logits.double() / temperature
    ordered, order = torch.sort(scaled, dim=-1, descending=True, stable=True)
    weights = torch.exp(ordered - ordered[:, :1])
    cumulative = torch.cumsum(weights, dim=-1)
    target = (p * cumulative[:, -1:]).contiguous()
    lengths = torch.searchsorted(cumulative.contiguous(), target, right=False).squeeze(-1) + 1
    return order.contiguous(), lengths.clamp(max=logits.shape[1]).to(torch.int64)


def sharded_topk_gpu(logits: torch.Tensor, k: int, shards: int, per_shard: int) -> torch.Tensor:
    """Untrusted approximate top-k (the fault model of `pck.faults.sharded_topk`; the role of
    the reference's `cuda/sampling.py:124-136`): a logit is a candidate if it ranks among the
    ``per_shard`` largest of its shard (equal shards, ties to the lower index); the result is
    the k largest candidates, ties to the lower index.  Exact when per_shard >= k."""
    rows, vocab = logits.shape
    if vocab % shards or per_shard > vocab // shards or k > shards * per_shard:
        raise ValueError("need vocab % shards == 0, per_shard <= vocab / shards, k <= pool")
    width = vocab // shards
    by_shard = logits.reshape(rows, shards, width)
    order = torch.sort(by_shard, dim=-1, descending=True, stable=True).indices
    rank = torch.empty_like(order).scatter_(
        -1, order, torch.arange(width, device=logits.device).expand_as(order)
    )
    candidate = (rank < per_shard).reshape(rows, vocab)
    masked = torch.where(candidate, logits, torch.full_like(logits, -float("inf")))
    return torch.sort(masked, dim=-1, descending=True, stable=True).indices[:, :k].contiguous()
