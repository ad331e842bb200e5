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


READ_CHUNK = 64 << 10  # bytes per workgroup of the read stream (fastest measured on MI355X)


def read_stream_ms(sizes: list[int], total: int = 1 << 30, reps: int = 20) -> list[float]:
    """Mean time of one `pck_read_stream` launch over ``sizes[i]`` bytes: enough buffers of
    each size to span ``total`` bytes (more than L2 + MALL) are read one after another from a
    captured HIP graph, so every launch streams from HBM and the host launch rate plays no part
    (the GEMV passes it is compared with are graph replays too).  The read-only ceiling of a
    launch of that many bytes."""
    from pck.cuda._lib import check, lib

    handle = lib()
    out = []
    for size in sizes:
        size = size // 16 * 16
        bufs = [torch.ones(size, dtype=torch.uint8, device="cuda") for _ in range(max(1, -(-total // size)))]
        groups = max(1, -(-size // READ_CHUNK))
        sink = torch.empty(4 * groups, dtype=torch.int32, device="cuda")

        def read_all() -> None:
            stream = torch.cuda.current_stream().cuda_stream
            for src in bufs:
                err = handle.pck_read_stream(src.data_ptr(), size, sink.data_ptr(), groups, stream)
                check(err, "read stream")

        read_all()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            read_all()
        graph.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        out.append(start.elapsed_time(end) / (reps * len(bufs)))
        del graph, bufs
    return out


def read_bandwidth_gbps(nbytes: int = 2 << 30, reps: int = 20) -> float:
    """Read-only streaming bandwidth of `pck_read_stream` over one 2 GiB buffer (larger than
    L2 + MALL): the long-stream HBM read ceiling."""
    (ms,) = read_stream_ms([nbytes], total=nbytes, reps=reps)
    return nbytes / (ms / 1e3) / 1e9
