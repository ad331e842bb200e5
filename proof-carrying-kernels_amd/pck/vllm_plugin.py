"""Checking every token vLLM samples, as a vLLM general plugin (drop-in for the reference's
`src/pck/vllm_plugin.py`: the same entry point, environment variables, wrapped method and
JSON-lines schema).

vLLM calls `register` in every process that loads the ``vllm.general_plugins`` entry points;
nothing happens unless ``PCK_CHECK_SAMPLING=1``.  Then the V2 model runner's sampler method
``vllm.v1.worker.gpu.sample.sampler.Sampler._sample_random`` (vLLM 0.33) is wrapped so that
each step's sampled tokens are checked against their rows of logits and their requests'
top-k / top-p / greedy settings.

Per step, on the device and without a host synchronisation:

1. the logits are copied before the sampler runs (vLLM's non-fused path masks them in place);
2. one launch of the HIP membership kernel (`pck.member.launch_check`) checks every row: it
   reads greedy from vLLM's per-request temperatures through the row's request index, takes
   top-p in the sampler's own precision and top-k's limit from vLLM's host copy, and adds the
   step's counts into a device buffer of running totals (rows, rejected, injected, caught,
   false alarms, and the largest r - p of an accepted top-p sample, kept as an
   order-preserving integer key so integer atomics suffice).

Every ``PCK_CHECK_EVERY`` steps the totals are copied to pinned host memory behind an event;
copies that have landed are written as JSON lines at later intervals (so the decode loop never
waits), and the rest at exit.

Environment (the reference's names and defaults):
  PCK_CHECK_SAMPLING=1   enable the check
  PCK_CHECK_LOG          JSON-lines file (default: pck_sampling_check.jsonl)
  PCK_CHECK_EVERY        steps between lines (default 16)
  PCK_CHECK_TOL          the sampler's own top-p tolerance (default 1e-4)
  PCK_FAULT_RATE         fault injection for testing the check: each constrained row (top-k,
                         top-p or greedy) is, with this probability, given its lowest-logit
                         token instead, where that token is truly outside the allowed set
                         (default 0: no injection, no extra launches)
"""

from __future__ import annotations

import atexit
import collections
import json
import os
import time
from dataclasses import dataclass
from pathlib import Path
from typing import Any

from pck.member import EXCESS_NONE, excess_value, launch_check, new_totals

COUNTS = ("rows", "rejected", "injected", "caught", "false_alarms")
"""The totals' integer fields, in the order of the JSON lines (reference
`src/pck/vllm_plugin.py:47`)."""


@dataclass(frozen=True)
class Snapshot:
    """A copy of the totals on its way to the host."""

    host: Any  # pinned (6,) int64
    ready: Any  # torch.cuda.Event recorded after the copy
    steps: int
    taken: float  # wall-clock time of the copy


class CheckStats:
    """The running totals of one worker process (reference name, `src/pck/vllm_plugin.py:38`).

    The counts live in a 6-word device buffer that the membership kernel adds each row into;
    `record_step` only counts steps on the host.  Snapshots of the buffer queue up behind
    events; `drain` writes every snapshot that has landed, in order, without waiting.  A line
    is {rows, rejected, injected, caught, false_alarms, steps, max_excess, seconds, pid, rank}:
    max_excess is the largest r - p over accepted top-p samples (-1: none), seconds the time
    since the stats were created, rank vLLM's RANK (or LOCAL_RANK) or null."""

    def __init__(self, path: Path, every: int) -> None:
        if every < 1:
            raise ValueError(f"every must be positive, got {every}")
        self.path = Path(path)
        self.every = every
        self.steps = 0
        self.written_steps = 0
        self.totals: Any = None  # device buffer, made on the first step's device
        self.queue: collections.deque[Snapshot] = collections.deque()
        self.start = time.time()
        self.pid = os.getpid()
        self.rank = os.environ.get("RANK", os.environ.get("LOCAL_RANK"))

    def buffer(self, device: Any) -> Any:
        """The device totals, made (zero counts, no excess) on first use."""
        if self.totals is None:
            self.totals = new_totals(device)
        return self.totals

    def record_step(self) -> None:
        """One checked step has been launched; at every ``every`` steps, write what has landed
        and queue a new snapshot."""
        self.steps += 1
        if self.steps % self.every == 0:
            self.drain(block=False)
            self.snapshot()

    def snapshot(self) -> None:
        """Queue a copy of the current totals to the host (no wait)."""
        import torch

        if self.totals is None:
            return
        host = torch.empty(6, dtype=torch.int64, pin_memory=True)
        host.copy_(self.totals, non_blocking=True)
        ready = torch.cuda.Event()
        ready.record(torch.cuda.current_stream(self.totals.device))
        self.queue.append(Snapshot(host, ready, self.steps, time.time()))

    def drain(self, block: bool) -> None:
        """Write the queued snapshots that have landed (all of them, waiting, with ``block``)."""
        while self.queue:
            snap = self.queue[0]
            if not snap.ready.query():
                if not block:
                    return
                snap.ready.synchronize()
            self.queue.popleft()
            self.write_line(snap)

    def line(self, snap: Snapshot) -> dict[str, Any]:
        words = snap.host.tolist()
        return {
            **{name: int(v) for name, v in zip(COUNTS, words[:5], strict=True)},
            "steps": snap.steps,
            "max_excess": excess_value(words[5] % 2**64),
            "seconds": round(snap.taken - self.start, 1),
            "pid": self.pid,
            "rank": self.rank,
        }

    def write_line(self, snap: Snapshot) -> None:
        with self.path.open("a") as f:
            f.write(json.dumps(self.line(snap)) + "\n")
        self.written_steps = snap.steps

    def flush(self) -> None:
        """Write everything: the queued snapshots, then the current totals if newer (waits for
        the device; registered to run at exit)."""
        self.drain(block=True)
        if self.totals is not None and self.written_steps != self.steps:
            self.snapshot()
            self.drain(block=True)


def plant_faults(logits: Any, tokens: Any, top_k: Any, top_p: Any, greedy: Any, tol: float,
                 top_k_host: Any, rate: float) -> tuple[Any, Any]:  # fmt: skip
    """(tokens with faults planted, injected mask): each row whose request is constrained
    (greedy, a top-k below V or a top-p below 1) is, with probability ``rate``, given its
    lowest-logit token, but only where the check itself finds that token outside the allowed
    set (ties at the bottom of a top-k, or top-p within tol of 1, allow it)."""
    import torch

    rows, vocab = logits.shape
    worst = logits.argmin(dim=1)
    outside = ~launch_check(logits, worst, top_k, top_p, greedy, tol, top_k_host)["ok"]
    constrained = greedy.clone()
    if top_k is not None:
        constrained |= top_k.reshape(rows) < vocab
    if top_p is not None:
        constrained |= top_p.reshape(rows) < 1.0
    drawn = torch.rand(rows, device=logits.device) < rate
    injected = drawn & constrained & outside
    return torch.where(injected, worst.to(tokens.dtype), tokens), injected


def install(
    sampler_cls: Any, log: Path, every: int = 16, tol: float = 1e-4, fault_rate: float = 0.0
) -> CheckStats:
    """Wrap ``sampler_cls._sample_random`` (vLLM 0.33's V2 sampler, or a stand-in with its
    signature) with the check; returns the stats, flushed at exit."""
    stats = CheckStats(log, every)
    sample = sampler_cls._sample_random

    def checked_sample_random(
        self: Any,
        processed_logits: Any,
        expanded_idx_mapping: Any,
        idx_mapping_np: Any,
        pos: Any,
        top_k: Any,
        top_p: Any,
        has_topp_only_rows: bool,
        use_fused_sampler: bool,
    ) -> tuple[Any, Any]:
        logits = processed_logits.clone()
        sampled, out = sample(
            self, processed_logits, expanded_idx_mapping, idx_mapping_np, pos, top_k, top_p,
            has_topp_only_rows, use_fused_sampler,
        )  # fmt: skip
        states = self.sampling_states
        rows = logits.shape[0]
        host = getattr(states, "top_k", None)  # vLLM's host copy of top-k: no sync
        top_k_host = host.np[idx_mapping_np] if host is not None and top_k is not None else None
        tokens, injected = sampled.reshape(rows), None
        if fault_rate > 0:
            greedy = states.temperature.gpu[expanded_idx_mapping] == 0
            tokens, injected = plant_faults(
                logits, tokens, top_k, top_p, greedy, tol, top_k_host, fault_rate
            )
            sampled = tokens.reshape(sampled.shape)
        launch_check(
            logits, tokens, top_k, top_p, None, tol, top_k_host,
            temperature=states.temperature.gpu, temperature_index=expanded_idx_mapping,
            injected=injected, totals=stats.buffer(logits.device), outputs=False,
        )  # fmt: skip
        stats.record_step()
        return sampled, out

    sampler_cls._sample_random = checked_sample_random
    atexit.register(stats.flush)
    return stats


@dataclass(frozen=True)
class Settings:
    """The plugin's environment (reference `src/pck/vllm_plugin.py:14-21`)."""

    enabled: bool
    log: Path
    every: int
    tol: float
    fault_rate: float

    @classmethod
    def from_env(cls, env: Any = None) -> Settings:
        env = os.environ if env is None else env
        return cls(
            enabled=env.get("PCK_CHECK_SAMPLING") == "1",
            log=Path(env.get("PCK_CHECK_LOG", "pck_sampling_check.jsonl")),
            every=int(env.get("PCK_CHECK_EVERY", "16")),
            tol=float(env.get("PCK_CHECK_TOL", "1e-4")),
            fault_rate=float(env.get("PCK_FAULT_RATE", "0")),
        )


def register() -> None:
    """vLLM's general-plugin entry point (``pck_sampling_check``): installs the check when
    ``PCK_CHECK_SAMPLING=1``; otherwise it does nothing and imports nothing from vLLM."""
    settings = Settings.from_env()
    if not settings.enabled:
        return
    from vllm.v1.worker.gpu.sample import sampler as vllm_sampler

    install(vllm_sampler.Sampler, settings.log, settings.every, settings.tol, settings.fault_rate)


__all__ = ["COUNTS", "EXCESS_NONE", "CheckStats", "Settings", "install", "plant_faults", "register"]
