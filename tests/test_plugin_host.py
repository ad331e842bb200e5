"""Host logic of the vLLM plugin and of the membership totals, without a GPU: the environment
settings and their defaults, `register` doing nothing (and importing no vLLM) unless enabled,
the order-preserving key of r - p the kernel's atomic maximum keeps, the initial totals, and
the JSON line a snapshot becomes (the reference's schema and key order)."""

from __future__ import annotations

import json
import math
import sys
import types
from pathlib import Path

import numpy as np
import pytest
import torch

from pck import vllm_plugin
from pck.member import EXCESS_NONE, excess_key, excess_value, key_as_int64, new_totals
from pck.vllm_plugin import COUNTS, CheckStats, Settings, Snapshot


def test_settings_defaults_and_overrides() -> None:
    s = Settings.from_env({})
    assert (s.enabled, s.log, s.every, s.tol, s.fault_rate) == (
        False, Path("pck_sampling_check.jsonl"), 16, 1e-4, 0.0,
    )  # fmt: skip
    s = Settings.from_env({"PCK_CHECK_SAMPLING": "1", "PCK_CHECK_LOG": "/tmp/x.jsonl",
                           "PCK_CHECK_EVERY": "4", "PCK_CHECK_TOL": "1e-3", "PCK_FAULT_RATE": "0.25"})  # fmt: skip
    assert (s.enabled, s.log, s.every, s.tol, s.fault_rate) == (True, Path("/tmp/x.jsonl"), 4, 1e-3, 0.25)
    assert not Settings.from_env({"PCK_CHECK_SAMPLING": "yes"}).enabled  # only "1" enables


def test_register_is_inert_unless_enabled(monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.delenv("PCK_CHECK_SAMPLING", raising=False)
    monkeypatch.setitem(sys.modules, "vllm", None)  # any import of vLLM would raise
    vllm_plugin.register()


def test_register_installs_on_vllms_sampler(monkeypatch: pytest.MonkeyPatch, tmp_path: Path) -> None:
    class Sampler:
        def _sample_random(self, *args):  # type: ignore[no-untyped-def]
            return args

    mod = types.ModuleType("vllm.v1.worker.gpu.sample.sampler")
    mod.Sampler = Sampler  # type: ignore[attr-defined]
    for name in ("vllm", "vllm.v1", "vllm.v1.worker", "vllm.v1.worker.gpu", "vllm.v1.worker.gpu.sample"):
        monkeypatch.setitem(sys.modules, name, types.ModuleType(name))
    monkeypatch.setitem(sys.modules, "vllm.v1.worker.gpu.sample.sampler", mod)
    sys.modules["vllm.v1.worker.gpu.sample"].sampler = mod  # type: ignore[attr-defined]
    monkeypatch.setenv("PCK_CHECK_SAMPLING", "1")
    monkeypatch.setenv("PCK_CHECK_LOG", str(tmp_path / "c.jsonl"))
    original = Sampler._sample_random
    vllm_plugin.register()
    assert Sampler._sample_random is not original
    assert Sampler._sample_random.__name__ == "checked_sample_random"


def test_excess_keys_order_and_round_trip() -> None:
    rng = np.random.default_rng(0)
    vals = sorted(set([-1.0, -0.5, -1e-300, -0.0, 1e-300, 0.25, 1.0] + list(rng.uniform(-1, 1, 200))))
    keys = [excess_key(v) for v in vals]
    assert keys == sorted(keys) and len(set(keys)) == len(keys)  # -0.0 sorts below +0.0
    for v in vals:
        back = excess_value(excess_key(v))
        assert back == v and math.copysign(1, back) == math.copysign(1, v)
    assert excess_key(0.0) == 1 << 63 and excess_key(-0.0) == (1 << 63) - 1


def test_new_totals() -> None:
    t = new_totals("cpu")
    assert t.dtype == torch.int64 and t.tolist()[:5] == [0] * 5
    assert excess_value(t.tolist()[5] % 2**64) == EXCESS_NONE


class Landed:
    """An event whose copy has completed."""

    def query(self) -> bool:
        return True

    def synchronize(self) -> None:
        pass


def test_snapshot_lines_keep_the_schema(tmp_path: Path, monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.setenv("RANK", "3")
    stats = CheckStats(tmp_path / "c.jsonl", every=2)
    host = torch.tensor([10, 3, 2, 2, 1, key_as_int64(excess_key(-0.015625))], dtype=torch.int64)
    stats.queue.append(Snapshot(host, Landed(), 2, stats.start + 1.04))
    stats.drain(block=False)
    line = json.loads((tmp_path / "c.jsonl").read_text())
    assert list(line) == [*COUNTS, "steps", "max_excess", "seconds", "pid", "rank"]
    assert line == {"rows": 10, "rejected": 3, "injected": 2, "caught": 2, "false_alarms": 1,
                    "steps": 2, "max_excess": -0.015625, "seconds": 1.0, "pid": stats.pid,
                    "rank": "3"}  # fmt: skip
    assert stats.written_steps == 2 and not stats.queue
    with pytest.raises(ValueError, match="every"):
        CheckStats(tmp_path / "d.jsonl", every=0)
