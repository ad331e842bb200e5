"""The detection campaign (`campaign.py`, the reference's protocol of harness/campaign.py and
harness/numerics_sim.py) at reduced size: honest outputs of both GEMV trees raise no alarm at
K = 8 for any activation family; bit-flip detection rises with the bit position and catches
every flip of exponent bit 30; every planted shortcut is caught at K = 8 and b <= 128, at
batch 1 (BF16 and FP8 weights, every Llama-3-8B projection) and on the batched down
projection; escapes at b = 256 are the smallest faults (BF16-rounded outputs or partial sums)
and pass only with |rho| <= tau."""

from __future__ import annotations

import pytest
import torch

import campaign

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def test_no_false_alarm_at_eight_draws() -> None:
    for block in (128, 64):
        print(f"false alarms b={block} K=8", flush=True)
        res = campaign.false_alarms(block, checks=8, target=200_000, redraw=8, seed=3)
        for kernel, r in res.items():
            assert r["block_checks"] >= 200_000
            assert r["alarms"] == 0, (block, kernel)
            assert set(r["by_family"]) == set(campaign.FAMILIES)
            assert 0 < r["max_rho_over_tau"] < 0.05, (block, kernel, r)


def test_bit_flip_rates_rise_with_the_bit() -> None:
    res = campaign.bit_flips(trials=16, seed=4, blocks=(64,), families=("gauss", "outliers"),
                             checks_list=(1,))  # fmt: skip
    bits = res["bits"]
    for family, cell in res["rates"]["b64"].items():
        rates = dict(zip(bits, cell["K1"]))
        print(family, rates, flush=True)
        assert rates[30] == 1.0  # the top exponent bit: a factor 2^128 or 2^-128
        assert rates[12] <= 0.05 <= rates[16] <= rates[20] <= rates[22]
        assert min(rates[23], rates[27], rates[31]) >= 0.95


def _check_shortcuts(summary: dict, strict_blocks: tuple[str, ...]) -> None:
    for case, per_block in summary.items():
        for bkey, row in per_block.items():
            assert row["false_alarms"] == 0, (case, bkey)
            kinds = {k: v for k, v in row.items() if k not in ("escapes", "false_alarms")}
            assert set(kinds) == set(campaign.SHORTCUTS + campaign.FLIPS), (case, bkey)
            if bkey in strict_blocks:
                for kind, frac in kinds.items():
                    caught, total = map(int, frac.split("/"))
                    assert caught == total, (case, bkey, kind, row["escapes"])
            for kind, ratios in row["escapes"].items():
                assert kind in ("bf16_output", "bf16_partials"), (case, bkey, kind)
                assert all(r <= 1.0 for r in ratios)


def test_every_shortcut_caught_at_eight_draws_batch_one() -> None:
    print("shortcuts K=8 batch 1", flush=True)
    summary = campaign.summarize_shortcuts(campaign.shortcuts_b1(seed=5))
    print(summary, flush=True)
    _check_shortcuts(summary, ("b64", "b128"))


def test_every_shortcut_caught_at_eight_draws_batched_down() -> None:
    print("shortcuts K=8 batched down projection", flush=True)
    summary = campaign.summarize_shortcuts(campaign.shortcuts_batched(seed=6, batches=(64,)))
    print(summary, flush=True)
    _check_shortcuts(summary, ("b64", "b128"))
