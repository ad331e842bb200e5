"""GEMV entry points (reference `src/pck/cuda/gemv.py:17-58`), backed by libpck_hip.so.

Same names, arguments, outputs and error behaviour as the reference: inputs are validated in
the order and with the messages of `src/pck/cuda/csrc/bindings.cpp:45-71` (RuntimeError), the
FP32 output is allocated on W's device and the kernel is enqueued on the current stream
without synchronising.
"""

from __future__ import annotations

import ctypes
from collections.abc import Sequence
from typing import Any

import torch

from pck.cuda._lib import MAX_GROUP, PckGemv, check, lib, stream_handle

INT32_MAX = 2**31 - 1
_NAMES = {torch.bfloat16: "BFloat16", torch.float8_e4m3fn: "Float8_e4m3fn"}


def _validate(
    W: torch.Tensor, x: torch.Tensor, threads: int, min_threads: int, w_type: torch.dtype
) -> None:
    if not (W.is_cuda and x.is_cuda):
        raise RuntimeError("W and x must be CUDA tensors")
    if W.device != x.device:
        raise RuntimeError("W and x must be on the same device")
    if W.dtype != w_type or x.dtype != torch.bfloat16:
        raise RuntimeError(f"W must be {_NAMES[w_type]} and x bfloat16")
    if not (W.dim() == 2 and x.dim() == 1 and x.size(0) == W.size(1)):
        raise RuntimeError(
            "expected W of shape (m, n) and x of shape (n,), got "
            f"{list(W.shape)} and {list(x.shape)}"
        )
    if not (W.is_contiguous() and x.is_contiguous()):
        raise RuntimeError("W and x must be contiguous")
    if not (min_threads <= threads <= 1024 and threads & (threads - 1) == 0):
        raise RuntimeError(
            f"threads must be a power of two in [{min_threads}, 1024], got {threads}"
        )
    if W.size(0) > INT32_MAX:
        raise RuntimeError("too many rows")


def _launch(
    entry: str, W: torch.Tensor, x: torch.Tensor, threads: int, min_threads: int,
    w_type: torch.dtype,
) -> torch.Tensor:  # fmt: skip
    _validate(W, x, threads, min_threads, w_type)
    handle = lib()
    y = torch.empty(W.size(0), dtype=torch.float32, device=W.device)
    if W.size(0) == 0:
        return y
    if W.size(1) == 0:
        raise RuntimeError("n must be positive")
    with torch.cuda.device(W.device):
        err = getattr(handle, entry)(
            W.data_ptr(), x.data_ptr(), y.data_ptr(), W.size(0), W.size(1), threads,
            stream_handle(W.device),
        )  # fmt: skip
    check(err, "gemv kernel launch")
    return y


def gemv_naive(W: torch.Tensor, x: torch.Tensor, threads: int = 256) -> torch.Tensor:
    """y = W x for contiguous BF16 tensors, FP32 accumulation and output, in the naive tree
    (contiguous chunk per lane): bit for bit the CPU model ``emulate_gemv`` with the same
    ``threads`` (reference `src/pck/cuda/gemv.py:17-24`)."""
    return _launch("pck_gemv_bf16_naive", W, x, threads, 1, torch.bfloat16)


def gemv_coalesced(W: torch.Tensor, x: torch.Tensor, threads: int = 256) -> torch.Tensor:
    """y = W x with 16-byte loads in the coalesced tree, ``threads`` a power of two in
    [32, 1024]: bit for bit ``emulate_gemv_coalesced(W, x, threads)`` (reference
    `src/pck/cuda/gemv.py:27-34`)."""
    return _launch("pck_gemv_bf16_coalesced", W, x, threads, 32, torch.bfloat16)


FP8_MAX = 448.0
"""Largest finite E4M3FN value."""


def quantize_fp8(W: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(Q, s) for `gemv_fp8`: one FP32 scale per row, s = max |w| / 448 (1 for an all-zero
    row), Q = clamp(W / s, +-448) cast to float8_e4m3fn (reference `src/pck/cuda/gemv.py:41-48`).
    Weight-load preparation in torch ops, as the reference's: the division by the scalar 448 is
    torch's product with the FP32 reciprocal, W / s is the IEEE FP32 quotient, and the cast
    rounds to the nearest E4M3 value, ties to even."""
    amax = W.abs().amax(dim=1).float()
    s = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    Q = (W.float() / s[:, None]).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return Q.contiguous(), s


def gemv_fp8(Q: torch.Tensor, x: torch.Tensor, threads: int = 256) -> torch.Tensor:
    """z = Q x for E4M3FN weights and BF16 x, FP32 accumulation and output, 16 weights per
    16-byte load: bit for bit ``emulate_gemv_coalesced(Q, x, threads, vec=16)``.  The row scales
    of `quantize_fp8` are applied by the caller afterwards, y = s z, so the checker verifies z
    against Q itself (reference `src/pck/cuda/gemv.py:51-58`)."""
    return _launch("pck_gemv_fp8_coalesced", Q, x, threads, 32, torch.float8_e4m3fn)


def _group_descriptors(
    pairs: Sequence[tuple[torch.Tensor, torch.Tensor]], threads: int
) -> tuple[ctypes.Array, list[torch.Tensor], int, torch.device]:  # type: ignore[type-arg]
    if not 1 <= len(pairs) <= MAX_GROUP:
        raise RuntimeError(f"group size must be in [1, {MAX_GROUP}], got {len(pairs)}")
    w_type = pairs[0][0].dtype
    if w_type not in _NAMES:
        raise RuntimeError("W must be BFloat16 or Float8_e4m3fn")
    device = pairs[0][0].device
    descs = (PckGemv * MAX_GROUP)()
    outs = []
    for g, (W, x) in enumerate(pairs):
        _validate(W, x, threads, 32, w_type)
        if W.device != device:
            raise RuntimeError("all GEMVs of a group must be on one device")
        if W.size(0) > 0 and W.size(1) == 0:
            raise RuntimeError("n must be positive")
        y = torch.empty(W.size(0), dtype=torch.float32, device=device)
        descs[g] = PckGemv(W.data_ptr(), x.data_ptr(), y.data_ptr(), W.size(0), W.size(1))
        outs.append(y)
    return descs, outs, (0 if w_type == torch.bfloat16 else 1), device


def gemv_group_check(
    pairs: Sequence[tuple[torch.Tensor, torch.Tensor]],
    checks: Sequence[tuple[Any, torch.Tensor, torch.Tensor]],
    threads: int = 256,
) -> tuple[list[torch.Tensor], list[Any]]:
    """`gemv_group` plus, in the same launch, the blocked checks of ``checks`` (up to eight
    ``(GpuBlockedChecker, x, y)`` items whose outputs came from earlier launches on this
    stream).  Returns the GEMV outputs and one `CheckResult` per check, bit-identical to
    ``check_many(checks)``.  The checker runs in its own workgroups of the launch and reads y
    from memory; its latency hides behind the GEMV stream.  No reference counterpart (the
    reference's checks are always a separate launch)."""
    from pck.cuda.checker import batch_for

    descs, outs, kind, device = _group_descriptors(pairs, threads)
    ride = None
    results: list[Any] = []
    if checks:
        ride, results, check_device = batch_for(checks)
        if check_device != device:
            raise RuntimeError("the checks must be on the GEMVs' device")
    with torch.cuda.device(device):
        err = lib().pck_gemv_group_check(
            kind, descs, len(pairs), threads, None if ride is None else ctypes.byref(ride),
            stream_handle(device),
        )  # fmt: skip
    check(err, "grouped gemv launch")
    return outs, results


def gemv_group_fp8_scaled(
    triples: Sequence[tuple[torch.Tensor, torch.Tensor, torch.Tensor]],
    checks: Sequence[tuple[Any, torch.Tensor, torch.Tensor]] = (),
    threads: int = 256,
) -> tuple[list[torch.Tensor], list[torch.Tensor], list[Any]]:
    """FP8 GEMVs that dequantise in the same launch: up to eight ``(Q, x, s)`` with Q E4M3FN
    (m, n), x BF16 (n,) and s the (m,) FP32 row scales of `quantize_fp8`.  Returns
    (z, y, check results): z = Q x with exactly the bits of `gemv_fp8` (what the checker
    verifies against Q), y = s z rounded as ``s * z`` rounds it, and, as in
    `gemv_group_check`, the results of ``checks`` carried in the launch.  No reference
    counterpart: the reference scales in a separate op after `gemv_fp8`
    (`src/pck/cuda/gemv.py:41-58`)."""
    from pck.cuda.checker import batch_for

    if not triples:
        raise RuntimeError(f"group size must be in [1, {MAX_GROUP}], got 0")
    pairs = [(Q, x) for Q, x, _ in triples]
    if any(Q.dtype != torch.float8_e4m3fn for Q, _ in pairs):
        raise RuntimeError("Q must be Float8_e4m3fn")
    descs, outs, _, device = _group_descriptors(pairs, threads)
    scales, scaled = [], []
    for (Q, _, sc) in triples:
        if not (sc.is_cuda and sc.device == device and sc.dtype == torch.float32 and sc.dim() == 1
                and sc.size(0) == Q.size(0) and sc.is_contiguous()):  # fmt: skip
            raise RuntimeError(f"s must be a contiguous ({Q.size(0)},) float32 tensor on {device}")
        scales.append(sc)
        scaled.append(torch.empty(Q.size(0), dtype=torch.float32, device=device))
    s_ptrs = (ctypes.c_void_p * len(triples))(*[t.data_ptr() for t in scales])
    y_ptrs = (ctypes.c_void_p * len(triples))(*[t.data_ptr() for t in scaled])
    ride = None
    results: list[Any] = []
    if checks:
        ride, results, check_device = batch_for(checks)
        if check_device != device:
            raise RuntimeError("the checks must be on the GEMVs' device")
    with torch.cuda.device(device):
        err = lib().pck_gemv_group_fp8_scaled(
            descs, s_ptrs, y_ptrs, len(triples), threads,
            None if ride is None else ctypes.byref(ride), stream_handle(device),
        )  # fmt: skip
    check(err, "grouped fp8 gemv launch")
    return outs, scaled, results


def gemv_fp8_scaled(
    Q: torch.Tensor, x: torch.Tensor, s: torch.Tensor, threads: int = 256
) -> tuple[torch.Tensor, torch.Tensor]:
    """(z, y) for one FP8 GEMV: z = Q x (the bits of `gemv_fp8`) and y = s z dequantised in the
    same launch."""
    z, y, _ = gemv_group_fp8_scaled([(Q, x, s)], (), threads)
    return z[0], y[0]


def gemv_group(
    pairs: Sequence[tuple[torch.Tensor, torch.Tensor]], threads: int = 256
) -> list[torch.Tensor]:
    """Several independent GEMVs of one weight type in one launch (e.g. q, k, v of a layer).

    ``pairs`` holds up to 8 ``(W, x)``; every W is BF16 (coalesced tree) or every W is
    E4M3FN (the FP8 tree).  Each output has exactly the bits `gemv_coalesced` or `gemv_fp8`
    would give.  No reference counterpart: the reference fuses such GEMVs by concatenating
    their weights (`harness/bench_decode_layer.py:48-53`).
    """
    descs, outs, kind, device = _group_descriptors(pairs, threads)
    with torch.cuda.device(device):
        err = lib().pck_gemv_group(kind, descs, len(pairs), threads, stream_handle(device))
    check(err, "grouped gemv launch")
    return outs


def gemv_group_rowsums(
    pairs: Sequence[tuple[torch.Tensor, torch.Tensor]],
    checks: Sequence[tuple[Any, torch.Tensor, torch.Tensor]] = (),
    threads: int = 256,
) -> tuple[list[torch.Tensor], list[torch.Tensor], list[Any]]:
    """In-pass GEMVs: `gemv_group` plus, for every GEMV, its row sums (m, 2) FP64
    (d_i = sum_j W_ij x_j and s_i = sum_j |W_ij x_j|, exact products, rounded-to-nearest sums in
    a fixed order) from the weights the launch streams anyway, and, in the same launch, the
    row-sum checks of ``checks``: up to eight ``(RowSumChecker, sums, y)`` items whose outputs
    came from earlier launches on this stream.  Returns (outputs, sums, check results); the
    outputs have exactly the bits of `gemv_group`, the results those of
    ``rowsum_check_many(checks)``.  No reference counterpart: the reference checks against a
    bank built at weight load (`src/pck/cuda/checker.py:91-104`)."""
    from pck.cuda.checker import rowsum_batch_for

    descs, outs, kind, device = _group_descriptors(pairs, threads)
    sums = [torch.empty((W.size(0), 2), dtype=torch.float64, device=device) for W, _ in pairs]
    ptrs = (ctypes.c_void_p * len(sums))(*[s.data_ptr() for s in sums])
    ride = None
    results: list[Any] = []
    if checks:
        ride, results, check_device = rowsum_batch_for(checks)
        if check_device != device:
            raise RuntimeError("the checks must be on the GEMVs' device")
    with torch.cuda.device(device):
        err = lib().pck_gemv_group_rowsums(
            kind, descs, ptrs, len(pairs), threads, None if ride is None else ctypes.byref(ride),
            stream_handle(device),
        )  # fmt: skip
    check(err, "in-pass gemv launch")
    return outs, sums, results


def gemv_coalesced_rowsums(
    W: torch.Tensor, x: torch.Tensor, threads: int = 256
) -> tuple[torch.Tensor, torch.Tensor]:
    """(y, sums): `gemv_coalesced` and the row sums of the in-pass launch."""
    _validate(W, x, threads, 32, torch.bfloat16)
    outs, sums, _ = gemv_group_rowsums([(W, x)], (), threads)
    return outs[0], sums[0]


def gemv_fp8_rowsums(
    Q: torch.Tensor, x: torch.Tensor, threads: int = 256
) -> tuple[torch.Tensor, torch.Tensor]:
    """(z, sums): `gemv_fp8` and the row sums of the in-pass launch (of Q itself, unscaled)."""
    _validate(Q, x, threads, 32, torch.float8_e4m3fn)
    outs, sums, _ = gemv_group_rowsums([(Q, x)], (), threads)
    return outs[0], sums[0]
