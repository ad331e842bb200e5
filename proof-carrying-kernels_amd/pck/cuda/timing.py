"""Benchmark timing with cold caches (reference `src/pck/cuda/timing.py`).

MI355X keeps a 256 MB Infinity Cache (MALL) behind its per-XCD L2s, and every Llama-3-8B
projection fits in it, so a flush of 2 x L2 (the reference's) would report MALL bandwidth as
HBM bandwidth.  `ColdL2Timer` keeps the reference's name and interface but overwrites at least
2 x (L2 + MALL) before every rep.
"""

from __future__ import annotations

import re
import statistics
from collections.abc import Callable
from dataclasses import dataclass

import torch

MALL_BYTES = 256 << 20
"""MI355X Infinity Cache (AMD's published size); torch does not report it."""


def device_name() -> str:
    """The GPU's model name without a trailing form-factor suffix."""
    return re.sub(r"\s+\w+ GPU$", "", torch.cuda.get_device_name())


def cache_bytes(device: int | torch.device = 0) -> int:
    """L2 as torch reports it plus the MALL."""
    props = torch.cuda.get_device_properties(device)
    return int(getattr(props, "L2_cache_size", 64 << 20)) + MALL_BYTES


@dataclass
class Timing:
    median_ms: float
    p10_ms: float
    p90_ms: float


class ColdL2Timer:
    """Times a GPU function with events, flushing L2 and the MALL before every rep."""

    def __init__(self, warmup: int, reps: int) -> None:
        self.flush = torch.empty(2 * cache_bytes(), dtype=torch.uint8, device="cuda")
        self.warmup, self.reps = warmup, reps

    def __call__(self, fn: Callable[[], object]) -> Timing:
        for _ in range(self.warmup):
            fn()
        starts = [torch.cuda.Event(enable_timing=True) for _ in range(self.reps)]
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(self.reps)]
        for start, end in zip(starts, ends, strict=True):
            self.flush.zero_()
            start.record()
            fn()
            end.record()
        torch.cuda.synchronize()
        times = sorted(float(s.elapsed_time(e)) for s, e in zip(starts, ends, strict=True))
        deciles = statistics.quantiles(times, n=10)
        return Timing(statistics.median(times), deciles[0], deciles[-1])


def copy_bandwidth_gbps(timer: ColdL2Timer, nbytes: int = 1 << 30) -> float:
    """Device-to-device copy bandwidth (read + write) (reference `timing.py:50-55`)."""
    src = torch.empty(nbytes // 2, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    t = timer(lambda: dst.copy_(src))
    return float(2 * src.numel() / (t.median_ms / 1e3) / 1e9)


def read_bandwidth_gbps(nbytes: int = 2 << 30, reps: int = 20) -> float:
    """Read-only streaming bandwidth of the `pck_read_stream` kernel over a buffer larger
    than L2 + MALL: the practical HBM read ceiling of the GEMVs."""
    from pck.cuda._lib import check, lib, stream_handle

    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    src.fill_(1)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    groups = 8 * cus
    sink = torch.empty(groups, dtype=torch.int32, device="cuda")

    def run() -> None:
        check(
            lib().pck_read_stream(
                src.data_ptr(), nbytes, sink.data_ptr(), groups, stream_handle(src.device)
            ),
            "read stream",
        )

    for _ in range(3):
        run()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        run()
    end.record()
    torch.cuda.synchronize()
    return nbytes * reps / (start.elapsed_time(end) / 1e3) / 1e9
