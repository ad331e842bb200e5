"""The vLLM plugin against a stand-in sampler with vLLM 0.33's method signature (the
reference's tests/test_vllm_plugin.py), on GPU tensors so every check runs the HIP kernel."""

from __future__ import annotations

import json
import os
from pathlib import Path
from types import SimpleNamespace
from typing import Any

import numpy as np
import pytest
import torch

from pck.vllm_plugin import install

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


class FakeSampler:
    """Samples a correct token per row (argmax for greedy rows, else uniform among vLLM's top-k
    survivors) and masks the logits in place as vLLM's non-fused path does."""

    def __init__(self, temperature: Any) -> None:
        self.sampling_states = SimpleNamespace(temperature=SimpleNamespace(gpu=temperature))

    def _sample_random(self, logits: Any, idx: Any, idx_np: Any, pos: Any, top_k: Any, top_p: Any, *_: Any):  # type: ignore[no-untyped-def]
        dev = logits.device
        k = top_k if top_k is not None else torch.full((logits.shape[0],), logits.shape[1], device=dev)
        kth = logits.topk(int(k.max()), dim=1).values.gather(1, (k - 1).reshape(-1, 1))
        logits.masked_fill_(logits < kth, -float("inf"))
        greedy = self.sampling_states.temperature.gpu[idx] == 0
        noise = torch.rand(logits.shape, device=dev)
        drawn = torch.where(torch.isfinite(logits), noise, -1.0).argmax(dim=1)
        return torch.where(greedy, logits.argmax(dim=1), drawn), logits


def batch(rows: int = 32, vocab: int = 200) -> tuple[Any, ...]:
    rng = np.random.default_rng(0)
    logits = torch.tensor(rng.standard_normal((rows, vocab)), dtype=torch.float32).cuda()
    idx = torch.arange(rows).cuda()
    top_k = torch.tensor(rng.choice([5, 20, vocab], rows)).cuda()
    return logits, idx, idx.cpu().numpy(), idx, top_k, None, False, True


def lines(path: Path) -> list[dict[str, Any]]:
    return [json.loads(line) for line in path.read_text().splitlines()]


def test_correct_samples_pass(tmp_path: Path) -> None:
    temperature = torch.tensor([0.0] * 4 + [1.0] * 28).cuda()
    cls = type("S", (FakeSampler,), {})
    log = tmp_path / "check.jsonl"
    stats = install(cls, log, every=1)
    for _ in range(3):
        cls(temperature)._sample_random(*batch())
    stats.flush()
    last = lines(log)[-1]
    assert last["steps"] == 3 and last["rows"] == 96 and last["rejected"] == 0


def test_injected_faults_are_all_caught_and_nothing_else(tmp_path: Path) -> None:
    cls = type("S", (FakeSampler,), {})
    log = tmp_path / "check.jsonl"
    stats = install(cls, log, every=1, fault_rate=0.5)
    for _ in range(4):
        cls(torch.ones(32).cuda())._sample_random(*batch())
    stats.flush()
    last = lines(log)[-1]
    assert last["injected"] > 0 and last["caught"] == last["injected"]
    assert last["false_alarms"] == 0 and last["rejected"] == last["injected"]


def test_top_p_rows_and_the_host_top_k_copy(tmp_path: Path) -> None:
    cls = type("S", (FakeSampler,), {})
    log = tmp_path / "check.jsonl"
    stats = install(cls, log, every=1, fault_rate=0.3)
    logits, idx, idx_np, pos, top_k, _, *rest = batch()
    top_p = torch.where(top_k < logits.shape[1], 0.999, 1.0)
    sampler = cls(torch.ones(32).cuda())
    sampler.sampling_states.top_k = SimpleNamespace(np=top_k.cpu().numpy())
    for _ in range(4):
        sampler._sample_random(logits.clone(), idx, idx_np, pos, top_k, top_p, *rest)
    stats.flush()
    last = lines(log)[-1]
    assert last["injected"] > 0 and last["caught"] == last["injected"]
    assert last["false_alarms"] == 0 and -1 <= last["max_excess"] < 0


def test_a_short_run_is_flushed_with_its_process_id(tmp_path: Path) -> None:
    cls = type("S", (FakeSampler,), {})
    log = tmp_path / "check.jsonl"
    stats = install(cls, log, every=100)
    for _ in range(3):
        cls(torch.ones(32).cuda())._sample_random(*batch())
    assert not log.exists()
    stats.flush()
    last = lines(log)[-1]
    assert last["steps"] == 3 and last["rows"] == 96 and last["pid"] == os.getpid()
    stats.flush()
    assert len(lines(log)) == 1


def test_faults_count_only_where_the_lowest_token_is_really_outside(tmp_path: Path) -> None:
    cls = type("S", (FakeSampler,), {})
    log = tmp_path / "check.jsonl"
    stats = install(cls, log, every=1, fault_rate=1.0)
    logits, idx, idx_np, pos, _, _, *rest = batch()
    loose = torch.full((32,), 0.99995).cuda()
    cls(torch.ones(32).cuda())._sample_random(logits, idx, idx_np, pos, None, loose, *rest)
    stats.flush()
    last = lines(log)[-1]
    assert last["injected"] == 0 and last["false_alarms"] == 0 and last["rejected"] == 0


def test_on_the_gpu_writes_lag_one_interval_and_flush_catches_up(tmp_path: Path) -> None:
    cls = type("S", (FakeSampler,), {})
    log = tmp_path / "check.jsonl"
    stats = install(cls, log, every=2)
    logits, idx, idx_np, pos, top_k, *rest = batch()
    for _ in range(5):
        cls(torch.ones(32).cuda())._sample_random(logits.clone(), idx, idx_np, pos, top_k, *rest)
    torch.cuda.synchronize()
    stats.flush()
    steps = [line["steps"] for line in lines(log)]
    assert steps[-1] == 5 and all(s in (2, 4, 5) for s in steps)
    assert lines(log)[-1]["rows"] == 160 and lines(log)[-1]["rejected"] == 0
