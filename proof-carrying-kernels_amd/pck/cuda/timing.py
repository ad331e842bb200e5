"""Benchmark timing with cold caches (reference `src/pck/cuda/timing.py`).

MI355X keeps a 256 MB Infinity Cache (MALL) behind its per-XCD L2s, and every Llama-3-8B
projection fits in it, so a flush of 2 x L2 (the reference's) would report MALL bandwidth as
HBM bandwidth.  `ColdL2Timer` keeps the reference's name and interface and scrubs
2 x (L2 + MALL) before every rep.
"""

from __future__ import annotations

import re
from collections.abc import Callable
from dataclasses import dataclass

import numpy as np
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
    """Times a GPU function rep by rep with events on the current stream, each rep starting
    from caches that hold none of its data (the reference's `ColdL2Timer` interface:
    ``ColdL2Timer(warmup, reps)(fn) -> Timing``).

    Before every rep a fill kernel writes a fresh byte value over a scrub buffer of
    2 x (L2 + MALL) bytes, so every line the previous rep left in L2 or the MALL has been
    replaced by the time the rep starts.  The reps are enqueued back to back and read after one
    synchronisation; the summary is the 10th, 50th and 90th percentiles of the rep times
    (linear interpolation between order statistics).
    """

    def __init__(self, warmup: int, reps: int) -> None:
        if warmup < 0 or reps < 1:
            raise ValueError(f"need warmup >= 0 and reps >= 1, got {warmup}, {reps}")
        self.warmup, self.reps = warmup, reps
        self._scrub = torch.empty(2 * cache_bytes(), dtype=torch.uint8, device="cuda")
        self._fill = 0

    @property
    def flush(self) -> torch.Tensor:
        """The scrub buffer written before every rep."""
        return self._scrub

    def _scrub_caches(self) -> None:
        self._fill = (self._fill + 1) % 256
        self._scrub.fill_(self._fill)

    def __call__(self, fn: Callable[[], object]) -> Timing:
        for _ in range(self.warmup):
            fn()
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(2 * self.reps)]
        for rep in range(self.reps):
            self._scrub_caches()
            marks[2 * rep].record()
            fn()
            marks[2 * rep + 1].record()
        marks[-1].synchronize()
        ms = np.array([marks[2 * r].elapsed_time(marks[2 * r + 1]) for r in range(self.reps)])
        p10, p50, p90 = np.percentile(ms, [10.0, 50.0, 90.0])
        return Timing(median_ms=float(p50), p10_ms=float(p10), p90_ms=float(p90))


def copy_bandwidth_gbps(timer: ColdL2Timer, nbytes: int = 1 << 30) -> float:
    """Device-to-device copy bandwidth, a practical DRAM ceiling (the reference's
    `copy_bandwidth_gbps` figure): one ``nbytes`` buffer whose first half is copied onto its
    second half, so every rep reads nbytes / 2 and writes nbytes / 2; bytes moved per second of
    the median rep."""
    half = nbytes // 2
    buf = torch.empty(2 * half, dtype=torch.uint8, device="cuda")
    src, dst = buf[:half], buf[half:]
    t = timer(lambda: dst.copy_(src))
    return float(2 * half / (t.median_ms * 1e-3) / 1e9)


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
