"""Trusted blocked checksum checker on the GPU (reference `src/pck/cuda/checker.py`).

The checksum bank (secret signs r, FP32 checksums c = r^T W_beta, and a_beta = sum |W_i|
rounded up to BF16) is built once at weight load.  In production the fault model is
non-adversarial, so signs drawn ahead of time are fine; an adversarial evaluation must draw
them after the untrusted kernel has finished.  The check itself is one launch of the HIP
kernel `pck_blocked_check` for up to eight GEMV outputs.
"""

from __future__ import annotations

import ctypes
import math
from collections.abc import Sequence
from dataclasses import dataclass
from typing import Any

import torch

from pck.cuda._lib import (
    MAX_BATCH,
    PckBatchCheckDesc,
    PckCheckBatch,
    PckCheckDesc,
    PckRowSumBatch,
    PckRowSumCheckDesc,
    check,
    lib,
    stream_handle,
)
from pck.fp import U32, U64, ceil_div, gamma, next_up, sum_up_factor

DEFAULT_BLOCK = 128
"""Rows per checksum (reference `src/pck/cuda/checker.py:20-22`)."""

KERNEL_THREADS = 256  # lanes per workgroup of the checker kernel
BLOCKS_PER_SM = 4  # workgroups per CU the default segment count aims for
MIN_SEGMENT_COLUMNS = 2 * KERNEL_THREADS

_DTYPE_NAMES = {
    torch.float32: "Float",
    torch.float64: "Double",
    torch.bfloat16: "BFloat16",
    torch.int8: "Char",
    torch.int32: "Int",
    torch.int64: "Long",
    torch.uint8: "Byte",
    torch.bool: "Bool",
    torch.float16: "Half",
}


def _dtype_name(dtype: torch.dtype) -> str:
    return _DTYPE_NAMES.get(dtype, str(dtype).removeprefix("torch."))


def round_up_bf16(v: torch.Tensor) -> torch.Tensor:
    """Non-negative FP64 values to BF16, never rounded down (reference
    `src/pck/cuda/checker.py:29-43`): up to FP32 first, then up to BF16 by carrying into the
    top 16 bits whenever a low bit is set.  Values past the BF16 range become +Inf."""
    if v.dtype != torch.float64:
        raise TypeError(f"round_up_bf16 expects float64, got {v.dtype}")
    if bool((v < 0).any()):
        raise ValueError("round_up_bf16 expects non-negative values")
    f = v.float()
    f = torch.where(f.double() < v, torch.nextafter(f, torch.full_like(f, math.inf)), f)
    bits = f.view(torch.int32)
    bits = torch.where((bits & 0xFFFF) != 0, (bits + 0x10000) & -0x10000, bits)
    return bits.view(torch.float32).to(torch.bfloat16)  # exact: the low 16 bits are zero


@dataclass(frozen=True)
class CheckResult:
    """Per (check, block) outcome; each tensor has shape (checks, num_blocks)."""

    passed: torch.Tensor
    rho: torch.Tensor
    tau: torch.Tensor

    @property
    def verdict(self) -> torch.Tensor:
        """Per-block verdict: True only if the block passed every check."""
        return self.passed.all(dim=0)


class GpuBlockedChecker:
    """Checks y = W x one block of ``block`` rows at a time, with ``checks`` sign draws
    (reference `src/pck/cuda/checker.py:60-137`).

    ``height`` is the summation-tree height of the GEMV being checked (e.g.
    ``tree_height(n, threads, vec)``).  ``segments`` and the scratch arrays keep the reference's
    interface and validation (default about ``BLOCKS_PER_SM`` workgroups per CU); the HIP
    kernel gives each (check, block) pair one workgroup over all n columns, so the value does
    not change the launch, and the result does not depend on it.  Use a checker from one stream
    at a time, as in the reference.
    """

    def __init__(
        self,
        W: torch.Tensor,
        block: int,
        height: int,
        checks: int = 1,
        generator: torch.Generator | None = None,
        segments: int | None = None,
    ) -> None:
        if not (W.is_cuda and W.dtype == torch.bfloat16 and W.dim() == 2):
            raise ValueError("W must be a 2-D bfloat16 CUDA tensor")
        m, n = W.shape
        if block < 1 or m % block:
            raise ValueError(f"block={block} must be positive and divide m={m}")
        if checks < 1:
            raise ValueError(f"checks must be positive, got {checks}")
        self.m, self.n, self.block, self.checks = m, n, block, checks
        self.num_blocks = m // block

        # Signs from a CPU generator, as the reference draws them (the same generator state
        # gives the same signs).
        bits = torch.randint(0, 2, (checks, self.num_blocks, block), generator=generator)
        self.r = (2 * bits - 1).to(torch.int8).to(W.device)

        W64 = W.view(self.num_blocks, block, n).double()
        c = torch.empty((checks, self.num_blocks, n), dtype=torch.float32, device=W.device)
        for k in range(checks):  # one draw at a time bounds the FP64 temporaries
            c[k] = torch.einsum("bi,bin->bn", self.r[k].double(), W64).float()
        self.c = c

        # The FP64 column sum rounds to nearest: lift it to an upper bound, then round up.
        col = W64.abs().sum(dim=1) * sum_up_factor(block)
        self.a = round_up_bf16(torch.nextafter(col, torch.full_like(col, math.inf)))
        del W64
        if not bool(torch.isfinite(self.a).all()):
            raise ValueError("sum of |W| over a block overflows BF16")

        self.coef = next_up(gamma(height) + U32, 2)
        if segments is None:
            cus = torch.cuda.get_device_properties(W.device).multi_processor_count
            wanted = ceil_div(BLOCKS_PER_SM * cus, checks * self.num_blocks)
            segments = max(1, min(wanted, n // MIN_SEGMENT_COLUMNS))
        if not 1 <= segments <= min(n, 65535):
            raise ValueError(f"segments must be in [1, {min(n, 65535)}], got {segments}")
        self.segments = segments
        # geps keeps the reference's form: the FP32 Dot2 chain term of its kernel
        # (gamma_2L(u32)^2, L terms per chain) and the FP64 height H of rho's evaluation,
        # compounded.  The HIP kernel evaluates rho in FP64 with exact products, whose error
        # gamma_H(u64) (sum |c_j x_j| + sum |y|) is within the gH term alone.
        chain = ceil_div(ceil_div(n, segments), KERNEL_THREADS)
        g2 = gamma(2 * chain, U32) ** 2
        fp64_height = max(n + block + 1, 21 + segments + ceil_div(block, KERNEL_THREADS))
        gh = gamma(fp64_height, U64)
        self.geps = next_up(gh + g2 + gh * g2, 4)
        self.tau_floor = next_up(n * 2.0**-148, 2)
        scratch = (checks, self.num_blocks, segments)
        self._partial_cx = torch.empty(scratch, dtype=torch.float64, device=W.device)
        self._partial_s = torch.empty(scratch, dtype=torch.float64, device=W.device)
        self._counters = torch.zeros((checks, self.num_blocks), dtype=torch.int32, device=W.device)

    def check(self, x: torch.Tensor, y: torch.Tensor) -> CheckResult:
        """Run every check on output ``y`` of the GEMV for input ``x``."""
        return check_many([(self, x, y)])[0]

    def verdict(self, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        """Per-block pass/fail (True = passed every check)."""
        return self.check(x, y).verdict

    def check_batched(self, X: torch.Tensor, Y: torch.Tensor) -> CheckResult:
        """Check every column of ``Y = X W^T`` (X (B, n) BF16, Y (B, m) FP32); results of
        shape (checks, num_blocks, B)."""
        return check_batched([(self, X, Y)])[0]


MAX_BATCH_CHECKS = MAX_BATCH


def _check_tensor(t: torch.Tensor, name: str, dtype: torch.dtype, device: torch.device) -> None:
    if not (t.is_cuda and t.device == device):
        raise RuntimeError(f"{name} must be on {device}")
    if t.dtype != dtype:
        raise RuntimeError(f"{name} must be {_dtype_name(dtype)}, got {_dtype_name(t.dtype)}")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _describe(
    c: torch.Tensor, a: torch.Tensor, r: torch.Tensor, x: torch.Tensor, y: torch.Tensor,
    partial_cx: torch.Tensor, partial_s: torch.Tensor, counters: torch.Tensor, coef: float,
    geps: float, tau_floor: float, device: torch.device,
) -> tuple[PckCheckDesc, tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:  # fmt: skip
    """Validates one check (reference `bindings.cpp:164-218`, same order and text) and
    returns its descriptor and freshly allocated outputs (passed, rho, tau)."""
    _check_tensor(c, "c", torch.float32, device)
    _check_tensor(a, "a", torch.bfloat16, device)
    _check_tensor(r, "r", torch.int8, device)
    _check_tensor(x, "x", torch.bfloat16, device)
    _check_tensor(y, "y", torch.float32, device)
    _check_tensor(partial_cx, "partial_cx", torch.float64, device)
    _check_tensor(partial_s, "partial_s", torch.float64, device)
    _check_tensor(counters, "counters", torch.int32, device)
    if not (c.dim() == 3 and a.dim() == 2 and r.dim() == 3 and x.dim() == 1 and y.dim() == 1):
        raise RuntimeError("expected c (K, nb, n), a (nb, n), r (K, nb, b), x (n,), y (m,)")
    checks, num_blocks, n = c.shape
    block = r.size(2)
    if not (a.size(0) == num_blocks and a.size(1) == n):
        raise RuntimeError("a must have shape (nb, n)")
    if not (r.size(0) == checks and r.size(1) == num_blocks):
        raise RuntimeError("r must have shape (K, nb, b)")
    if x.size(0) != n:
        raise RuntimeError("x must have shape (n,)")
    if y.size(0) != num_blocks * block:
        raise RuntimeError("y must have shape (nb * b,)")
    if not (checks >= 1 and num_blocks >= 1 and n >= 1 and block >= 1):
        raise RuntimeError("empty checker")
    if not (
        partial_cx.dim() == 3
        and partial_cx.size(0) == checks
        and partial_cx.size(1) == num_blocks
        and partial_s.shape == partial_cx.shape
    ):
        raise RuntimeError("partial sums must have shape (K, nb, segments)")
    if not (counters.dim() == 2 and counters.size(0) == checks and counters.size(1) == num_blocks):
        raise RuntimeError("counters must have shape (K, nb)")
    segments = partial_cx.size(2)
    if not 1 <= segments <= n:
        raise RuntimeError(f"segments must be in [1, n], got {segments}")
    if not (coef > 0 and geps > 0 and tau_floor > 0):
        raise RuntimeError("coef, geps and floor must be positive")
    shape = (checks, num_blocks)
    passed = torch.empty(shape, dtype=torch.bool, device=device)
    rho = torch.empty(shape, dtype=torch.float64, device=device)
    tau = torch.empty(shape, dtype=torch.float64, device=device)
    desc = PckCheckDesc(
        c.data_ptr(), a.data_ptr(), r.data_ptr(), x.data_ptr(), y.data_ptr(),
        partial_cx.data_ptr(), partial_s.data_ptr(), counters.data_ptr(), passed.data_ptr(),
        rho.data_ptr(), tau.data_ptr(), n, ceil_div(n, segments), block, num_blocks, checks,
        segments, coef, geps, tau_floor,
    )  # fmt: skip
    return desc, (passed, rho, tau)


def build_batch(
    c: Sequence[torch.Tensor], a: Sequence[torch.Tensor], r: Sequence[torch.Tensor],
    x: Sequence[torch.Tensor], y: Sequence[torch.Tensor], partial_cx: Sequence[torch.Tensor],
    partial_s: Sequence[torch.Tensor], counters: Sequence[torch.Tensor], coef: Sequence[float],
    geps: Sequence[float], tau_floor: Sequence[float],
) -> tuple[PckCheckBatch, list[tuple[torch.Tensor, torch.Tensor, torch.Tensor]], torch.device]:  # fmt: skip
    """Validates up to eight checks (reference `bindings.cpp:221-256`: same argument lists,
    order and messages) and returns the launch descriptor, the freshly allocated outputs
    (passed, rho, tau) of each check, and the device."""
    count = len(c)
    if not 1 <= count <= MAX_BATCH:
        raise RuntimeError(f"batch size must be in [1, {MAX_BATCH}], got {count}")
    lists = (a, r, x, y, partial_cx, partial_s, counters, coef, geps, tau_floor)
    if any(len(v) != count for v in lists):
        raise RuntimeError("all argument lists must have the same length")
    if not y[0].is_cuda:
        raise RuntimeError("y must be a CUDA tensor")
    device = y[0].device
    batch = PckCheckBatch()
    batch.count = count
    outputs = []
    for g in range(count):
        if not y[g].is_cuda:
            raise RuntimeError("y must be a CUDA tensor")
        desc, out = _describe(
            c[g], a[g], r[g], x[g], y[g], partial_cx[g], partial_s[g], counters[g], coef[g],
            geps[g], tau_floor[g], device,
        )  # fmt: skip
        batch.desc[g] = desc
        batch.start[g + 1] = batch.start[g] + desc.checks * desc.num_blocks  # one per pair
        outputs.append(out)
    if batch.start[count] > 2**31 - 1:
        raise RuntimeError("too many blocks")
    return batch, outputs, device


def blocked_check(
    c: Sequence[torch.Tensor], a: Sequence[torch.Tensor], r: Sequence[torch.Tensor],
    x: Sequence[torch.Tensor], y: Sequence[torch.Tensor], partial_cx: Sequence[torch.Tensor],
    partial_s: Sequence[torch.Tensor], counters: Sequence[torch.Tensor], coef: Sequence[float],
    geps: Sequence[float], tau_floor: Sequence[float],
) -> list[tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:  # fmt: skip
    """Checks up to eight GEMV outputs in one launch; (passed, rho, tau) per check.

    The native entry of the reference's extension (`bindings.cpp:221-256`): same argument
    lists, validation order and messages; the launch goes to `pck_blocked_check`.
    """
    batch, outputs, device = build_batch(
        c, a, r, x, y, partial_cx, partial_s, counters, coef, geps, tau_floor
    )
    with torch.cuda.device(device):
        err = lib().pck_blocked_check(batch, stream_handle(device))
    check(err, "checker kernel launch")
    return outputs


def batch_for(
    items: Sequence[tuple[GpuBlockedChecker, torch.Tensor, torch.Tensor]],
) -> tuple[PckCheckBatch, list[CheckResult], torch.device]:
    """Launch descriptor and result tensors for up to eight ``(checker, x, y)`` items."""
    if len({id(checker) for checker, _, _ in items}) != len(items):
        raise ValueError("each checker may appear only once per call")
    batch, outputs, device = build_batch(
        [ch.c for ch, _, _ in items],
        [ch.a for ch, _, _ in items],
        [ch.r for ch, _, _ in items],
        [x for _, x, _ in items],
        [y for _, _, y in items],
        [ch._partial_cx for ch, _, _ in items],
        [ch._partial_s for ch, _, _ in items],
        [ch._counters for ch, _, _ in items],
        [ch.coef for ch, _, _ in items],
        [ch.geps for ch, _, _ in items],
        [ch.tau_floor for ch, _, _ in items],
    )
    return batch, [CheckResult(*out) for out in outputs], device


def check_many(
    items: Sequence[tuple[GpuBlockedChecker, torch.Tensor, torch.Tensor]],
) -> list[CheckResult]:
    """Check several GEMV outputs, ``(checker, x, y)`` each, eight per launch (reference
    `src/pck/cuda/checker.py:143-171`).  Each checker may appear only once per call, since a
    launch uses its scratch."""
    if len({id(checker) for checker, _, _ in items}) != len(items):
        raise ValueError("each checker may appear only once per call")
    results: list[CheckResult] = []
    for i in range(0, len(items), MAX_BATCH):
        chunk = items[i : i + MAX_BATCH]
        outputs = blocked_check(
            [ch.c for ch, _, _ in chunk],
            [ch.a for ch, _, _ in chunk],
            [ch.r for ch, _, _ in chunk],
            [x for _, x, _ in chunk],
            [y for _, _, y in chunk],
            [ch._partial_cx for ch, _, _ in chunk],
            [ch._partial_s for ch, _, _ in chunk],
            [ch._counters for ch, _, _ in chunk],
            [ch.coef for ch, _, _ in chunk],
            [ch.geps for ch, _, _ in chunk],
            [ch.tau_floor for ch, _, _ in chunk],
        )
        results.extend(CheckResult(passed, rho, tau) for passed, rho, tau in outputs)
    return results


def rowsum_depth(n: int) -> int:
    """Depth D of the in-pass row sums of a row of n columns, for every launch: the most
    additions any term passes through, over thread counts 32..1024 and vectors of 8 or 16
    columns.  Lane l of min(T, 64) lanes adds (T / min(T, 64)) ceil(ceil(n / V) / T) V terms in
    sequence (padding included: adding +0 is exact; d takes them in pairs, half as many), then
    log2 min(T, 64) butterfly levels."""
    depth = 0
    for threads in (32, 64, 128, 256, 512, 1024):
        lanes = min(threads, 64)
        for vec in (8, 16):
            per_lane = (threads // lanes) * ceil_div(ceil_div(n, vec), threads) * vec
            depth = max(depth, per_lane + lanes.bit_length() - 1)
    return depth


class RowSumChecker:
    """Blocked checks of y = W x from the row sums of an in-pass GEMV launch, with no bank.

    The in-pass launch (`pck.cuda.gemv_group_rowsums`) writes, beside y, a pair per row from
    the FP32 products p_j = W_ij x_j the tree forms anyway: d_i (consecutive products added in
    pairs in FP32, the pair sums added in FP64) and s_i (sum of |p_j| in FP32).  The check
    then reads 16 bytes per row instead of the bank's 6n bytes per block (2.3% of BF16 and 4.7%
    of FP8 weight bytes at b = 128).  Each (check, block) pair is the blocked checker's
    relation (reference `src/pck/cuda/csrc/checker_kernel.cu:115-183`): rho = r . d_beta -
    r . y_beta, tau = coef s + geps ((1 + u32) s + sum |y|) + tau_floor, with s an upper bound
    of the exact S = sum |W_ij x_j| over the block.  Soundness (T2/T3): coef = gamma_h + u32 as
    in `GpuBlockedChecker`; gamma_h S covers the GEMV tree's error and u32 S the FP32 pair sums
    of d (at most u32 (|p0| + |p1|) each), as it covers the FP32 rounding of c there;
    ``s_factor`` = 1 + (D + 1) 2^-23 bounds the FP32 sums of |p| of depth D = `rowsum_depth`(n);
    ``geps`` = gamma_H(u64), H = D + ceil(b / 64) + 7, covers rho's FP64 evaluation; and
    ``tau_floor`` adds 2 b n 2^-150 for FP32 product underflow to the bank checker's n 2^-148.
    The resulting tau is within (1 + 2^-14) of the threshold for the exact S, where the bank's
    BF16 column sums a make it up to 2^-8 looser.  Signs come from the same draw as
    `GpuBlockedChecker` (the same generator state gives the same r).

    The check runs inside the producing GEMV's launch sequence: it suits the production
    (non-adversarial) fault model, as the bank checker with signs drawn at weight load does
    (reference `src/pck/cuda/checker.py:4-6`); the bank checker stays the trusted reference.
    """

    def __init__(
        self,
        m: int,
        n: int,
        block: int,
        height: int,
        checks: int = 1,
        generator: torch.Generator | None = None,
        device: torch.device | str | None = None,
    ) -> None:
        if block < 1 or m % block:
            raise ValueError(f"block={block} must be positive and divide m={m}")
        if checks < 1:
            raise ValueError(f"checks must be positive, got {checks}")
        if n < 1:
            raise ValueError(f"n must be positive, got {n}")
        device = torch.device("cuda") if device is None else torch.device(device)
        self.m, self.n, self.block, self.checks = m, n, block, checks
        self.num_blocks = m // block
        bits = torch.randint(0, 2, (checks, self.num_blocks, block), generator=generator)
        self.r = (2 * bits - 1).to(torch.int8).to(device)
        depth = rowsum_depth(n)
        self.coef = next_up(gamma(height) + U32, 2)
        self.geps = next_up(gamma(depth + ceil_div(block, 64) + 7, U64), 2)
        self.tau_floor = next_up(n * 2.0**-148 + 2 * block * n * 2.0**-150, 2)
        self.s_factor = next_up(1.0 + (depth + 1) * 2.0**-23, 2)

    @property
    def device(self) -> torch.device:
        return self.r.device

    def check(self, sums: torch.Tensor, y: torch.Tensor) -> CheckResult:
        """Run every check on output ``y`` with its row sums ``sums`` (m, 2) FP64."""
        return rowsum_check_many([(self, sums, y)])[0]

    def verdict(self, sums: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        """Per-block pass/fail (True = passed every check)."""
        return self.check(sums, y).verdict


def rowsum_batch_for(
    items: Sequence[tuple[RowSumChecker, torch.Tensor, torch.Tensor]],
) -> tuple[Any, list[CheckResult], torch.device]:
    """Validates up to eight ``(RowSumChecker, sums, y)`` items and returns the launch
    descriptor (a `PckRowSumBatch`), freshly allocated results and the device."""
    if not 1 <= len(items) <= MAX_BATCH:
        raise RuntimeError(f"batch size must be in [1, {MAX_BATCH}], got {len(items)}")
    device = items[0][0].device
    batch = PckRowSumBatch()
    batch.count = len(items)
    results = []
    for g, (ch, sums, y) in enumerate(items):
        _check_tensor(sums, "sums", torch.float64, device)
        _check_tensor(y, "y", torch.float32, device)
        if ch.device != device:
            raise RuntimeError(f"the checker's signs must be on {device}")
        if tuple(sums.shape) != (ch.m, 2):
            raise RuntimeError(f"sums must have shape ({ch.m}, 2), got {list(sums.shape)}")
        if tuple(y.shape) != (ch.m,):
            raise RuntimeError(f"y must have shape ({ch.m},), got {list(y.shape)}")
        if sums.data_ptr() % 16:
            raise RuntimeError("sums must be 16-byte aligned")
        shape = (ch.checks, ch.num_blocks)
        passed = torch.empty(shape, dtype=torch.bool, device=device)
        rho = torch.empty(shape, dtype=torch.float64, device=device)
        tau = torch.empty(shape, dtype=torch.float64, device=device)
        batch.desc[g] = PckRowSumCheckDesc(
            sums.data_ptr(), y.data_ptr(), ch.r.data_ptr(), passed.data_ptr(), rho.data_ptr(),
            tau.data_ptr(), ch.block, ch.num_blocks, ch.checks, 0, ch.coef, ch.geps,
            ch.tau_floor, ch.s_factor,
        )  # fmt: skip
        batch.start[g + 1] = batch.start[g] + ch.checks * ch.num_blocks
        results.append(CheckResult(passed, rho, tau))
    if batch.start[batch.count] > 2**31 - 1:
        raise RuntimeError("too many blocks")
    return batch, results, device


def rowsum_check_many(
    items: Sequence[tuple[RowSumChecker, torch.Tensor, torch.Tensor]],
) -> list[CheckResult]:
    """Row-sum checks of several outputs, ``(checker, sums, y)`` each, eight per launch
    (`pck_rowsum_check`).  A row-sum check uses no scratch, so a checker may appear more than
    once."""
    results: list[CheckResult] = []
    for i in range(0, len(items), MAX_BATCH):
        batch, res, device = rowsum_batch_for(items[i : i + MAX_BATCH])
        with torch.cuda.device(device):
            err = lib().pck_rowsum_check(batch, stream_handle(device))
        check(err, "row-sum check launch")
        results.extend(res)
    return results


def check_batched(
    items: Sequence[tuple[GpuBlockedChecker, torch.Tensor, torch.Tensor]],
) -> list[CheckResult]:
    """Check the outputs of batched products, ``(checker, X, Y)`` each with X (B, n) BF16 and
    Y (B, m) FP32 (``Y = X W^T``): every column of Y is checked as `check_many` checks one
    GEMV output, with the checker's bank, signs and constants (build the checker with the
    height of the batched product's tree).  Up to eight outputs per launch; results have
    shape (checks, num_blocks, B) (B = 0 gives empty results and launches nothing), and
    ``verdict`` is then (num_blocks, B).  No reference
    counterpart: the reference checks one vector per call (`src/pck/cuda/checker.py:143-171`).
    """
    out: dict[int, CheckResult] = {}
    for item in items:  # an empty batch: validated, nothing to launch
        if item[1].dim() == 2 and item[1].size(0) == 0:
            out[id(item)] = _describe_batched([item])[1][0]
    direct = [item for item in items if id(item) not in out and _batched_kernel_fits(*item)]
    for item in items:
        if id(item) not in out and not _batched_kernel_fits(*item):
            out[id(item)] = _check_columns(*item)
    for res, item in zip(_check_batched_direct(direct), direct):
        out[id(item)] = res
    return [out[id(item)] for item in items]


def _check_columns(ch: GpuBlockedChecker, X: torch.Tensor, Y: torch.Tensor) -> CheckResult:
    """Every column of Y checked as one GEMV output, up to eight columns per launch of the
    single-vector kernel, all against the same bank (this kernel uses no scratch, so one
    checker may fill several descriptors of a launch); results (checks, num_blocks, B)."""
    if not (X.dim() == 2 and Y.dim() == 2 and X.size(0) == Y.size(0)):
        raise RuntimeError("X must be (B, n) and Y (B, m) with the same B")
    cols = []
    for b0 in range(0, X.size(0), MAX_BATCH):
        xs = [X[b].contiguous() for b in range(b0, min(b0 + MAX_BATCH, X.size(0)))]
        ys = [Y[b].contiguous() for b in range(b0, min(b0 + MAX_BATCH, X.size(0)))]
        k = len(xs)
        batch, outputs, device = build_batch(
            [ch.c] * k, [ch.a] * k, [ch.r] * k, xs, ys, [ch._partial_cx] * k, [ch._partial_s] * k,
            [ch._counters] * k, [ch.coef] * k, [ch.geps] * k, [ch.tau_floor] * k,
        )  # fmt: skip
        with torch.cuda.device(device):
            err = lib().pck_blocked_check(batch, stream_handle(device))
        check(err, "checker kernel launch")
        cols.extend(outputs)
    return CheckResult(*(torch.stack([c[i] for c in cols], dim=-1) for i in range(3)))


def _batched_kernel_fits(ch: GpuBlockedChecker, X: torch.Tensor, Y: torch.Tensor) -> bool:
    """The batched kernel reads eight bank columns and four outputs per load: n % 8 == 0,
    block % 4 == 0 and 16-byte aligned X and Y (other shapes are checked column by column, with
    the same verdicts)."""
    return ch.n % 8 == 0 and ch.block % 4 == 0 and X.data_ptr() % 16 == 0 and Y.data_ptr() % 16 == 0


def batched_descriptors(
    chunk: Sequence[tuple[GpuBlockedChecker, torch.Tensor, torch.Tensor]],
) -> tuple[Any, list[CheckResult], torch.device]:
    """Validated launch descriptors (a `PckBatchCheckDesc` array) for up to eight
    ``(checker, X, Y)`` items, freshly allocated results, and the device."""
    descs, results, device = _describe_batched(chunk)
    if any(X.size(0) == 0 for _, X, _ in chunk):
        raise RuntimeError("batch size must be positive")
    return descs, results, device


def _describe_batched(
    chunk: Sequence[tuple[GpuBlockedChecker, torch.Tensor, torch.Tensor]],
) -> tuple[Any, list[CheckResult], torch.device]:
    """`batched_descriptors` without the batch-size rule: an item with B = 0 gets results of
    shape (checks, num_blocks, 0)."""
    descs = (PckBatchCheckDesc * len(chunk))()
    results: list[CheckResult] = []
    device = None
    for g, (ch, X, Y) in enumerate(chunk):
        if device is None:
            if not Y.is_cuda:
                raise RuntimeError("Y must be a CUDA tensor")
            device = Y.device
        _check_tensor(X, "X", torch.bfloat16, device)
        _check_tensor(Y, "Y", torch.float32, device)
        if ch.c.device != device:
            raise RuntimeError(f"the checker's bank must be on {device}")
        if not (X.dim() == 2 and X.size(1) == ch.n):
            raise RuntimeError(f"X must have shape (B, {ch.n}), got {list(X.shape)}")
        if not (Y.dim() == 2 and Y.size(0) == X.size(0) and Y.size(1) == ch.m):
            raise RuntimeError(f"Y must have shape ({X.size(0)}, {ch.m}), got {list(Y.shape)}")
        B = X.size(0)
        shape = (ch.checks, ch.num_blocks, B)
        passed = torch.empty(shape, dtype=torch.bool, device=device)
        rho = torch.empty(shape, dtype=torch.float64, device=device)
        tau = torch.empty(shape, dtype=torch.float64, device=device)
        results.append(CheckResult(passed, rho, tau))
        descs[g] = PckBatchCheckDesc(
            ch.c.data_ptr(), ch.a.data_ptr(), ch.r.data_ptr(), X.data_ptr(), Y.data_ptr(),
            passed.data_ptr(), rho.data_ptr(), tau.data_ptr(), ch.n, ch.block,
            ch.num_blocks, ch.checks, B, ch.coef, ch.geps, ch.tau_floor,
        )  # fmt: skip
    assert device is not None
    return descs, results, device


def _check_batched_direct(
    items: Sequence[tuple[GpuBlockedChecker, torch.Tensor, torch.Tensor]],
) -> list[CheckResult]:
    results: list[CheckResult] = []
    for i in range(0, len(items), MAX_BATCH):
        chunk = items[i : i + MAX_BATCH]
        descs, res, device = batched_descriptors(chunk)
        results.extend(res)
        need = ctypes.c_int64(0)
        check(lib().pck_batch_check_workspace(descs, len(chunk), ctypes.byref(need)),
              "batched checker plan")  # fmt: skip
        work = torch.empty(max(1, need.value // 8), dtype=torch.float64, device=device)
        with torch.cuda.device(device):
            err = lib().pck_batch_check(descs, len(chunk), work.data_ptr(), need.value,
                                        stream_handle(device))  # fmt: skip
        check(err, "batched checker launch")
    return results


class PendingCheck:
    """A check running on a `SideStreamChecker`'s stream (reference name and use,
    `src/pck/cuda/checker.py:174-186`).  Its result tensors were allocated on the submitting
    stream, so `wait` there only orders that stream after the check's completion event."""

    def __init__(self, result: CheckResult, done: torch.cuda.Event, owner: torch.cuda.Stream) -> None:
        self._result = result
        self._done = done
        self._owner = owner

    def wait(self) -> CheckResult:
        """Make the current stream wait for the check and return its result."""
        current = torch.cuda.current_stream(self._owner.device)
        current.wait_event(self._done)
        if current != self._owner:  # keep the allocator from recycling them under this stream
            for t in (self._result.passed, self._result.rho, self._result.tau):
                t.record_stream(current)
        return self._result

    def done(self) -> bool:
        """Whether the check has finished (never waits)."""
        return bool(self._done.query())


class SideStreamChecker:
    """Runs blocked checks on a stream of its own (default priority), so a check overlaps the
    work the caller enqueues after it (reference name and use, `src/pck/cuda/checker.py:189-215`).

    `submit` validates and allocates on the caller's current stream, records an event there (so
    the check starts only after the kernel that produced y), and launches on the side stream;
    inputs and outputs are marked as used by the side stream for the allocator.  Checks on one
    side stream run in submission order, so a checker's state is never used by two at once.
    """

    def __init__(self, device: torch.device | None = None) -> None:
        self.stream = torch.cuda.Stream(device)

    def submit(self, checker: GpuBlockedChecker, x: torch.Tensor, y: torch.Tensor) -> PendingCheck:
        caller = torch.cuda.current_stream(self.stream.device)
        batch, (result,), device = batch_for([(checker, x, y)])
        produced = torch.cuda.Event()
        produced.record(caller)
        self.stream.wait_event(produced)
        for t in (x, y, result.passed, result.rho, result.tau):
            t.record_stream(self.stream)
        with torch.cuda.device(device):
            err = lib().pck_blocked_check(batch, int(self.stream.cuda_stream))
        check(err, "checker kernel launch")
        done = torch.cuda.Event()
        done.record(self.stream)
        return PendingCheck(result, done, caller)

    def wait_all(self) -> None:
        """Make the current stream wait for every check submitted so far."""
        torch.cuda.current_stream(self.stream.device).wait_stream(self.stream)


def carry_selection(checker_ids: Sequence[int], limit: int = MAX_BATCH) -> list[int]:
    """Positions of the queued checks one launch takes, oldest first: at most ``limit``, each
    checker at most once (a launch takes a checker's descriptor once, as `check_many`
    requires); a checker's later checks wait for a later launch."""
    taken: list[int] = []
    seen: set[int] = set()
    for i, cid in enumerate(checker_ids):
        if len(taken) == limit:
            break
        if cid not in seen:
            seen.add(cid)
            taken.append(i)
    return taken


class CarriedCheck:
    """A check queued on a `CarriedChecker`.  Its `CheckResult` exists once a launch has taken
    the check (a carrying GEMV launch or `CarriedChecker.flush`); the tensors fill in stream
    order, as every result of this module does."""

    def __init__(self) -> None:
        self._result: CheckResult | None = None

    @property
    def launched(self) -> bool:
        """Whether a launch has taken the check (its result tensors exist)."""
        return self._result is not None

    def result(self) -> CheckResult:
        """The check's result; raises if no launch has taken the check yet."""
        if self._result is None:
            raise RuntimeError(
                "the check has not been launched: issue a carrying GEMV launch through its "
                "CarriedChecker or call flush()"
            )
        return self._result


class CarriedChecker:
    """The reference's call pattern, GEMV launches and then `check_many` over their outputs
    (reference `src/pck/cuda/checker.py:143-171`), with the checks carried by later GEMV
    launches instead of a launch of their own.

    - `check_many(items)` (or `submit(checker, x, y)`) validates the checks and queues them;
      it returns one `CarriedCheck` per item.
    - `gemv_group(pairs)` (and `gemv_group_fp8_scaled(triples)`) issues the GEMVs.  A launch
      of at least ``min_rows`` rows also carries up to eight queued checks, oldest first
      (`pck_gemv_group_check`): its first workgroups run them while the rest stream the
      weights.  Smaller launches carry nothing: a launch that fits in one round of the GPU
      would wait for the CUs that host checks.
    - `flush()` runs whatever is still queued as standalone launches (`check_many`).

    Results are bit-identical to `check_many` on the same items.  A queued check's y must come
    from a launch issued earlier on the stream that carries it: the stream current at
    `submit` is recorded, and a launch on another stream refuses to carry the check.  Under
    graph capture the queue is host state of the capture, as every launch argument is.  No
    reference counterpart: the reference's checks are always a launch of their own.
    """

    def __init__(self, threads: int = 256, min_rows: int = 16384) -> None:
        self.threads = threads
        self.min_rows = min_rows
        self._queue: list[tuple[tuple[GpuBlockedChecker, torch.Tensor, torch.Tensor], CarriedCheck, torch.cuda.Stream]] = []  # fmt: skip

    @property
    def pending(self) -> int:
        """Checks queued and not yet launched."""
        return len(self._queue)

    def submit(self, checker: GpuBlockedChecker, x: torch.Tensor, y: torch.Tensor) -> CarriedCheck:
        """Queue one check of output ``y`` for input ``x``."""
        device = checker.c.device
        _check_tensor(x, "x", torch.bfloat16, device)
        _check_tensor(y, "y", torch.float32, device)
        if x.dim() != 1 or x.size(0) != checker.n:
            raise RuntimeError("x must have shape (n,)")
        if y.dim() != 1 or y.size(0) != checker.num_blocks * checker.block:
            raise RuntimeError("y must have shape (nb * b,)")
        handle = CarriedCheck()
        self._queue.append(((checker, x, y), handle, torch.cuda.current_stream(device)))
        return handle

    def check_many(
        self, items: Sequence[tuple[GpuBlockedChecker, torch.Tensor, torch.Tensor]]
    ) -> list[CarriedCheck]:
        """Queue ``(checker, x, y)`` items (`check_many`'s arguments)."""
        return [self.submit(checker, x, y) for checker, x, y in items]

    def _take(self, rows: int, device: torch.device) -> list[tuple[Any, CarriedCheck, torch.cuda.Stream]]:  # fmt: skip
        if rows < self.min_rows or not self._queue:
            return []
        picked = [self._queue[i] for i in carry_selection([id(e[0][0]) for e in self._queue])]
        stream = torch.cuda.current_stream(device)
        if any(e[2] != stream for e in picked):
            raise RuntimeError("a queued check was submitted on another stream than this launch's")
        return picked

    def _settle(self, picked: list[tuple[Any, CarriedCheck, Any]], results: Sequence[CheckResult]) -> None:  # fmt: skip
        for entry, result in zip(picked, results, strict=True):
            entry[1]._result = result
        taken = {id(e) for e in picked}
        self._queue = [e for e in self._queue if id(e) not in taken]

    def gemv_group(self, pairs: Sequence[tuple[torch.Tensor, torch.Tensor]]) -> list[torch.Tensor]:
        """`gemv_group(pairs)`, carrying queued checks when the launch is large enough."""
        from pck.cuda.gemv import gemv_group_check

        picked = self._take(sum(int(W.size(0)) for W, _ in pairs), pairs[0][0].device) if pairs else []
        ys, results = gemv_group_check(pairs, [e[0] for e in picked], self.threads)
        self._settle(picked, results)
        return ys

    def gemv_group_fp8_scaled(
        self, triples: Sequence[tuple[torch.Tensor, torch.Tensor, torch.Tensor]]
    ) -> tuple[list[torch.Tensor], list[torch.Tensor]]:
        """`gemv_group_fp8_scaled(triples)` (z and y = s z), carrying queued checks when the
        launch is large enough."""
        from pck.cuda.gemv import gemv_group_fp8_scaled

        picked = self._take(sum(int(Q.size(0)) for Q, _, _ in triples), triples[0][0].device) if triples else []  # fmt: skip
        zs, ys, results = gemv_group_fp8_scaled(triples, [e[0] for e in picked], self.threads)
        self._settle(picked, results)
        return zs, ys

    def flush(self) -> None:
        """Run every queued check now, in standalone launches on the current stream."""
        while self._queue:
            picked = [self._queue[i] for i in carry_selection([id(e[0][0]) for e in self._queue])]
            device = picked[0][0][0].c.device
            stream = torch.cuda.current_stream(device)
            if any(e[2] != stream for e in picked):
                raise RuntimeError("a queued check was submitted on another stream than this launch's")
            self._settle(picked, check_many([e[0] for e in picked]))
