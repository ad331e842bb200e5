"""Batched decode product Y = X W^T for B >= 16 activation rows on the matrix cores (libpck_hip).

No reference counterpart on the hot path: the reference's nearest code is the diagnostic
`harness/csrc/batched_gemv.cu:25-117` (B <= 8 on FP32 cores).  The kernel's order is fixed and
restated on the CPU by the oracle, so the outputs are bit-exact against it, and the tree height
that the blocked checker needs is `batched_height(n)`.

Two routes with the same bits:

- `gemm_batched(W, X)` with a plain (m, n) weight tensor runs the element kernel (any shape);
- `gemm_batched(pack_batched_weights(W), X)` runs the packed kernel: the weights are packed
  once, at load time, into 32-row tiles whose matrix-core operands are contiguous, and each call
  packs X the same way into a workspace.  This is the decode path.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from pck.cuda._lib import check, lib, stream_handle

STEP = 8
WAVES = 8
GROUP = 16  # chunks per group inside a K segment
TILE = 32
PAIR_COLUMNS = 128  # packed route: K segments of whole step pairs


def batched_height(n: int) -> int:
    """Tree height of one output of `gemm_batched`: 9 for a matrix-core step (8 truncated
    products, one rounding); for the longest K segment of P chunks, min(P, 16) additions inside
    a group of 16 chunks plus ceil(P / 16) adding the group sums; 3 for the segment tree."""
    chunks = max(1, math.ceil(n / STEP))
    per = math.ceil(chunks / WAVES)
    return 9 + min(per, GROUP) + math.ceil(per / GROUP) + int(math.log2(WAVES))


@dataclass
class BatchedWeights:
    """Weights for `gemm_batched` in the packed 32-row tile layout (`packed` is None when the
    shape has no packed route: n % 128 != 0 or m % 4 != 0; then `raw` is used)."""

    m: int
    n: int
    dtype: torch.dtype
    packed: torch.Tensor | None
    raw: torch.Tensor | None

    @property
    def device(self) -> torch.device:
        t = self.packed if self.packed is not None else self.raw
        assert t is not None
        return t.device


def _kind(dtype: torch.dtype) -> int:
    return 0 if dtype == torch.bfloat16 else 1


def _packable(m: int, n: int) -> bool:
    return n >= PAIR_COLUMNS and n % PAIR_COLUMNS == 0 and m % 4 == 0


def _pack(src: torch.Tensor, kind: int) -> torch.Tensor:
    rows, n = src.shape
    tiles = (rows + TILE - 1) // TILE
    elem = torch.uint8 if kind == 1 else torch.bfloat16
    dst = torch.empty(tiles * TILE * n, dtype=elem, device=src.device)
    with torch.cuda.device(src.device):
        err = lib().pck_bgemm_pack(kind, src.data_ptr(), dst.data_ptr(), rows, n,
                                   stream_handle(src.device))  # fmt: skip
    check(err, "batched pack launch")
    return dst


def _validate_w(W: torch.Tensor) -> None:
    if not W.is_cuda:
        raise RuntimeError("W must be a CUDA tensor")
    if W.dtype not in (torch.bfloat16, torch.float8_e4m3fn):
        raise RuntimeError("W must be BFloat16 or Float8_e4m3fn")
    if W.dim() != 2:
        raise RuntimeError(f"expected W of shape (m, n), got {list(W.shape)}")
    if not W.is_contiguous():
        raise RuntimeError("W must be contiguous")


def pack_batched_weights(W: torch.Tensor) -> BatchedWeights:
    """Packs W (m, n) BF16 or float8_e4m3fn (raw codes) once for the packed kernel; enqueued on
    the current stream.  Shapes without a packed route keep W as it is."""
    _validate_w(W)
    m, n = W.shape
    if m == 0 or not _packable(m, n):
        return BatchedWeights(m, n, W.dtype, None, W)
    return BatchedWeights(m, n, W.dtype, _pack(W, _kind(W.dtype)), None)


def gemm_batched(
    W: torch.Tensor | BatchedWeights, X: torch.Tensor, out: torch.Tensor | None = None
) -> torch.Tensor:
    """Y (B, m) FP32 = X (B, n) BF16 times W^T for W (m, n) BF16 or float8_e4m3fn (raw codes;
    row scales are the caller's, as for `gemv_fp8`), or W packed by `pack_batched_weights`.
    Enqueued on the current stream; written into ``out`` (a contiguous (B, m) float32 tensor on
    W's device) when given, so that a check of Y can be planned before the product runs."""
    packed = isinstance(W, BatchedWeights)
    if packed:
        m, n, dtype, device = W.m, W.n, W.dtype, W.device
    else:
        if not W.is_cuda:
            raise RuntimeError("W and X must be CUDA tensors")
        m, n = W.shape if W.dim() == 2 else (-1, -1)
        dtype, device = W.dtype, W.device
    if not X.is_cuda:
        raise RuntimeError("W and X must be CUDA tensors")
    if device != X.device:
        raise RuntimeError("W and X must be on the same device")
    if dtype not in (torch.bfloat16, torch.float8_e4m3fn) or X.dtype != torch.bfloat16:
        raise RuntimeError("W must be BFloat16 or Float8_e4m3fn and X bfloat16")
    if not packed and W.dim() != 2 or not (X.dim() == 2 and X.size(1) == n):
        raise RuntimeError(
            f"expected W of shape (m, n) and X of shape (B, n), got {[m, n]} and {list(X.shape)}"
        )
    if (not packed and not W.is_contiguous()) or not X.is_contiguous():
        raise RuntimeError("W and X must be contiguous")
    B = X.size(0)
    if out is None:
        Y = torch.empty((B, m), dtype=torch.float32, device=device)
    else:
        if not (out.is_cuda and out.device == device and out.dtype == torch.float32
                and out.shape == (B, m) and out.is_contiguous()):  # fmt: skip
            raise RuntimeError(f"out must be a contiguous ({B}, {m}) float32 tensor on {device}")
        Y = out
    if m == 0 or B == 0:
        return Y
    if n == 0:
        raise RuntimeError("n must be positive")
    kind = _kind(dtype)
    with torch.cuda.device(device):
        if packed and W.packed is not None:
            Xp = _pack(X, 0)
            err = lib().pck_bgemm_packed(kind, W.packed.data_ptr(), Xp.data_ptr(), Y.data_ptr(),
                                         m, n, B, stream_handle(device))  # fmt: skip
        else:
            raw = W.raw if packed else W
            assert raw is not None
            err = lib().pck_bgemm(kind, raw.data_ptr(), X.data_ptr(), Y.data_ptr(), m, n, B,
                                  stream_handle(device))  # fmt: skip
    check(err, "batched gemm launch")
    return Y
