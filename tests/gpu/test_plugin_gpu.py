"""The vLLM plugin (`pck.vllm_plugin`) on the GPU, driven by a scripted stand-in with vLLM
0.33's `_sample_random` signature.

- the device totals the membership kernel keeps equal the counts of the CPU oracle
  (`oracle.member.check_members_ref`) over every step: rows, rejected, and max_excess within the
  oracle's mass tolerance; rows are mapped to requests through a permuted index, so greediness
  is read through it;
- planted faults are all caught, with no false alarm, and only where the lowest-logit token is
  truly outside the allowed set;
- the logits the sampler masks in place are checked as they were before it ran;
- JSON lines keep the reference's schema and key order, are written after the copy lands, and
  flush writes the rest exactly once.
"""

from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace
from typing import Any

import numpy as np
import pytest
import torch

from oracle.member import check_members_ref
from pck.member import member_eps32
from pck.vllm_plugin import COUNTS, install

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

FIELDS = [*COUNTS, "steps", "max_excess", "seconds", "pid", "rank"]


class ScriptedSampler:
    """Returns the tokens it is given for each call and, like vLLM's non-fused path, masks the
    logits it receives in place (everything below each row's 3rd largest becomes -inf)."""

    def __init__(self, temperature: torch.Tensor, top_k_np: np.ndarray | None = None) -> None:
        states = SimpleNamespace(temperature=SimpleNamespace(gpu=temperature))
        if top_k_np is not None:
            states.top_k = SimpleNamespace(np=top_k_np)
        self.sampling_states = states
        self.script: list[torch.Tensor] = []

    def _sample_random(self, logits, idx, idx_np, pos, top_k, top_p, *_):  # type: ignore[no-untyped-def]
        tokens = self.script.pop(0)
        third = logits.topk(3, dim=1).values[:, 2:3]
        logits.masked_fill_(logits < third, -float("inf"))
        return tokens.clone(), logits


def lines(path: Path) -> list[dict[str, Any]]:
    return [json.loads(line) for line in path.read_text().splitlines()]


def step_inputs(seed: int, rows: int = 48, vocab: int = 3000):  # type: ignore[no-untyped-def]
    """Logits with a few hot tokens, per-row top-k (some none), top-p (some none) in FP32, and a
    mix of tokens: the argmax, a token just inside the top-k, one far outside, the minimum."""
    rng = np.random.default_rng(seed)
    logits = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    hot = rng.integers(0, vocab, (rows, 4))
    np.put_along_axis(logits, hot, np.take_along_axis(logits, hot, 1) + 12, 1)
    top_k = rng.choice([5, 50, vocab], rows)
    top_p = rng.choice([0.8, 0.95, 1.0], rows).astype(np.float32)
    order = np.argsort(-logits, axis=1, kind="stable")
    pick = rng.integers(0, 4, rows)
    choices = np.stack([order[:, 0], order[:, 3], order[:, 200], order[:, -1]], 1)
    tokens = choices[np.arange(rows), pick]
    return logits, top_k, top_p, tokens


def run_steps(tmp_path: Path, fault_rate: float = 0.0, every: int = 1, steps: int = 4,
              host_top_k: bool = False):  # type: ignore[no-untyped-def]  # fmt: skip
    rows = 48
    log = tmp_path / "check.jsonl"
    cls = type("S", (ScriptedSampler,), {})
    stats = install(cls, log, every=every, fault_rate=fault_rate)
    temperature = torch.ones(rows, device="cuda")
    expected_rejected = 0
    for step in range(steps):
        logits, top_k, top_p, tokens = step_inputs(100 + step)
        honest = np.argsort(-logits, axis=1, kind="stable")[:, 0]  # the argmax: always allowed
        use = honest if fault_rate > 0 else tokens
        ref = check_members_ref(logits, use, top_k, top_p.astype(np.float64), None, 1e-4)
        expected_rejected += int((~ref["ok"]).sum())
        sampler = cls(temperature, top_k if host_top_k else None)
        sampler.script.append(torch.from_numpy(use).cuda())
        idx = torch.arange(rows, device="cuda")
        sampler._sample_random(
            torch.from_numpy(logits).cuda(), idx, idx.cpu().numpy(), idx,
            torch.from_numpy(top_k).cuda(), torch.from_numpy(top_p).cuda(), False, False,
        )  # fmt: skip
    stats.flush()
    return stats, lines(log), expected_rejected


def test_counts_schema_and_flush(tmp_path: Path) -> None:
    stats, got, expected_rejected = run_steps(tmp_path, steps=4, every=1)
    assert [line["steps"] for line in got][-1] == 4
    assert all(list(line) == FIELDS for line in got)
    last = got[-1]
    assert last["rows"] == 4 * 48 and last["rejected"] == expected_rejected > 0
    assert last["false_alarms"] == last["rejected"] and last["injected"] == last["caught"] == 0
    assert isinstance(last["max_excess"], float) and -1.0 <= last["max_excess"] < 0.0
    before = len(got)
    stats.flush()  # nothing new: no second line for the same steps
    assert len(lines(stats.path)) == before


def test_oracle_counts_through_the_request_index(tmp_path: Path) -> None:
    rows, requests = 48, 64
    rng = np.random.default_rng(7)
    temperature = rng.choice([0.0, 0.7, 1.0], requests).astype(np.float32)
    idx = rng.permutation(requests)[:rows]  # row r serves request idx[r]
    log = tmp_path / "check.jsonl"
    cls = type("S", (ScriptedSampler,), {})
    stats = install(cls, log, every=3)
    sampler = cls(torch.from_numpy(temperature).cuda())
    rejected, excess = 0, -1.0
    for step in range(5):
        logits, top_k, top_p, tokens = step_inputs(step)
        greedy = temperature[idx] == 0
        ref = check_members_ref(logits, tokens, top_k, top_p.astype(np.float64), greedy, 1e-4)
        rejected += int((~ref["ok"]).sum())
        nucleus = ref["ok"] & (top_p < 1.0) & ~greedy
        if nucleus.any():
            excess = max(excess, float((ref["mass_above"] - top_p.astype(np.float64))[nucleus].max()))
        sampler.script.append(torch.from_numpy(tokens).cuda())
        t_idx = torch.from_numpy(idx).cuda()
        sampler._sample_random(
            torch.from_numpy(logits).cuda(), t_idx, idx, t_idx, torch.from_numpy(top_k).cuda(),
            torch.from_numpy(top_p).cuda(), False, False,
        )  # fmt: skip
    stats.flush()
    got = lines(log)
    assert [line["steps"] for line in got] == [3, 5]
    last = got[-1]
    assert last["rows"] == 5 * rows and last["rejected"] == rejected
    assert abs(last["max_excess"] - excess) <= 4 * member_eps32(3000)


def test_planted_faults_are_all_caught(tmp_path: Path) -> None:
    _, got, expected_rejected = run_steps(tmp_path, fault_rate=0.5, steps=6, host_top_k=True)
    last = got[-1]
    assert expected_rejected == 0  # the scripted tokens are argmaxes: all allowed
    assert last["injected"] > 0 and last["caught"] == last["injected"] == last["rejected"]
    assert last["false_alarms"] == 0


def test_no_fault_where_every_token_is_allowed(tmp_path: Path) -> None:
    """Top-p within tol of 1 and no top-k allows every token: nothing may be planted."""
    log = tmp_path / "check.jsonl"
    cls = type("S", (ScriptedSampler,), {})
    stats = install(cls, log, every=1, fault_rate=1.0)
    logits, _, _, tokens = step_inputs(5)
    loose = torch.full((48,), 0.99995, device="cuda")
    sampler = cls(torch.ones(48, device="cuda"))
    sampler.script.append(torch.from_numpy(tokens).cuda())
    idx = torch.arange(48, device="cuda")
    sampler._sample_random(torch.from_numpy(logits).cuda(), idx, idx.cpu().numpy(), idx, None,
                           loose, False, False)  # fmt: skip
    stats.flush()
    last = lines(log)[-1]
    assert last["injected"] == 0 and last["rejected"] == 0 and last["false_alarms"] == 0


def test_lines_follow_the_copies(tmp_path: Path) -> None:
    stats, got, _ = run_steps(tmp_path, every=2, steps=5)
    steps = [line["steps"] for line in got]
    assert steps == sorted(steps) and steps[-1] == 5 and set(steps) <= {2, 4, 5}
    assert got[-1]["rows"] == 5 * 48
