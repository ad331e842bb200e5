"""Batched decode product Y = X W^T for B >= 16 activation rows on the matrix cores (libpck_hip).

No reference counterpart on the hot path: the reference's nearest code is the diagnostic
`harness/csrc/batched_gemv.cu:25-117` (B <= 8 on FP32 cores).  The kernel's order is fixed and
restated on the CPU by the oracle, so the outputs are bit-exact against it, and the tree height
that the blocked checker needs is `batched_height(n)`.
"""

from __future__ import annotations

import math

import torch

from pck.cuda._lib import check, lib, stream_handle

STEP = 8
WAVES = 8


def batched_height(n: int) -> int:
    """Tree height of one output of `gemm_batched`: 9 for a matrix-core step (8 truncated
    products, one rounding), the longest K segment's additions, and 3 for the segment tree."""
    chunks = max(1, math.ceil(n / STEP))
    return 9 + math.ceil(chunks / WAVES) + int(math.log2(WAVES))


def gemm_batched(W: torch.Tensor, X: torch.Tensor) -> torch.Tensor:
    """Y (B, m) FP32 = X (B, n) BF16 times W^T for W (m, n) BF16 or float8_e4m3fn (raw codes;
    row scales are the caller's, as for `gemv_fp8`).  Enqueued on the current stream."""
    if not (W.is_cuda and X.is_cuda):
        raise RuntimeError("W and X must be CUDA tensors")
    if W.device != X.device:
        raise RuntimeError("W and X must be on the same device")
    if W.dtype not in (torch.bfloat16, torch.float8_e4m3fn) or X.dtype != torch.bfloat16:
        raise RuntimeError("W must be BFloat16 or Float8_e4m3fn and X bfloat16")
    if not (W.dim() == 2 and X.dim() == 2 and X.size(1) == W.size(1)):
        raise RuntimeError(
            f"expected W of shape (m, n) and X of shape (B, n), got {list(W.shape)} and "
            f"{list(X.shape)}"
        )
    if not (W.is_contiguous() and X.is_contiguous()):
        raise RuntimeError("W and X must be contiguous")
    m, n = W.shape
    B = X.size(0)
    Y = torch.empty((B, m), dtype=torch.float32, device=W.device)
    if m == 0 or B == 0:
        return Y
    if n == 0:
        raise RuntimeError("n must be positive")
    kind = 0 if W.dtype == torch.bfloat16 else 1
    with torch.cuda.device(W.device):
        err = lib().pck_bgemm(
            kind, W.data_ptr(), X.data_ptr(), Y.data_ptr(), m, n, B, stream_handle(W.device)
        )
    check(err, "batched gemm launch")
    return Y
