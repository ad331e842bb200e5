"""Host-side logic of the pck package that runs without a GPU: the validation the wrappers do
before any launch (same order and messages as the reference's bindings), the refusal to run
without the HIP library's device path, and round_up_bf16 (reference
tests/gpu/test_round_up_bf16.py runs on CPU tensors too).  The plugin's host logic is in
tests/test_plugin_host.py."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from hypothesis import given
from hypothesis import strategies as st

from pck.cuda import GpuBlockedChecker, check_many, gemv_coalesced, gemv_fp8, gemv_naive
from pck.cuda.checker import blocked_check, round_up_bf16
from pck.member import check_members

BF16_MAX = float(torch.finfo(torch.bfloat16).max)


@pytest.mark.parametrize("fn", [gemv_naive, gemv_coalesced])
def test_gemv_refuses_cpu_tensors(fn) -> None:  # type: ignore[no-untyped-def]
    W = torch.ones((4, 8), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="CUDA tensors"):
        fn(W, torch.ones(8, dtype=torch.bfloat16), 32)


def test_fp8_gemv_refuses_cpu_tensors() -> None:
    with pytest.raises(RuntimeError, match="CUDA tensors"):
        gemv_fp8(torch.zeros((4, 16), dtype=torch.float8_e4m3fn), torch.ones(16, dtype=torch.bfloat16))


def test_membership_refuses_cpu_logits() -> None:
    with pytest.raises(RuntimeError, match="on the GPU"):
        check_members(torch.zeros((2, 10)), torch.zeros(2, dtype=torch.long))


def test_checker_refuses_cpu_weights() -> None:
    with pytest.raises(ValueError, match="bfloat16 CUDA"):
        GpuBlockedChecker(torch.ones((8, 8), dtype=torch.bfloat16), 4, 4)


def test_check_many_rejects_duplicates_before_launch() -> None:
    fake = object()
    with pytest.raises(ValueError, match="once"):
        check_many([(fake, None, None), (fake, None, None)])  # type: ignore[list-item]


def test_blocked_check_rejects_bad_batches_before_launch() -> None:
    t = torch.zeros(1)
    with pytest.raises(RuntimeError, match="batch size"):
        blocked_check(*([] for _ in range(11)))
    with pytest.raises(RuntimeError, match="batch size"):
        blocked_check(*([t] * 9 for _ in range(11)))
    lists = [[t] for _ in range(11)]
    lists[4] = [t, t]
    with pytest.raises(RuntimeError, match="same length"):
        blocked_check(*lists)
    with pytest.raises(RuntimeError, match="CUDA"):
        blocked_check(*([t] for _ in range(11)))


@given(st.lists(st.floats(0, BF16_MAX, allow_nan=False), min_size=1, max_size=50))
def test_round_up_bf16_never_rounds_down_and_is_tight(values: list[float]) -> None:
    v = torch.tensor(values, dtype=torch.float64)
    up = round_up_bf16(v)
    assert up.dtype == torch.bfloat16
    up64 = up.double()
    assert bool((up64 >= v).all())
    # the next BF16 value below the result is below the input (or the result is zero)
    bits = up.view(torch.int16).numpy().astype(np.int32)
    below = torch.from_numpy((bits - 1).astype(np.int16)).view(torch.bfloat16).double().numpy()
    assert np.all((below < np.array(values)) | (up64.numpy() == 0))


@pytest.mark.parametrize(
    ("value", "expected"),
    [(0.0, 0.0), (1.0, 1.0), (1 + 2**-30, 1 + 2**-7), (1 + 2**-8, 1 + 2**-7), (3.0, 3.0)],
)
def test_round_up_bf16_known_values(value: float, expected: float) -> None:
    assert float(round_up_bf16(torch.tensor([value], dtype=torch.float64))[0]) == expected


def test_round_up_bf16_overflow_and_errors() -> None:
    assert math.isinf(float(round_up_bf16(torch.tensor([BF16_MAX * 1.001], dtype=torch.float64))[0]))
    with pytest.raises(ValueError, match="non-negative"):
        round_up_bf16(torch.tensor([-1.0], dtype=torch.float64))
    with pytest.raises(TypeError, match="float64"):
        round_up_bf16(torch.tensor([1.0]))




def test_carry_selection_takes_each_checker_once_oldest_first() -> None:
    from pck.cuda.checker import carry_selection

    assert carry_selection([]) == []
    assert carry_selection([7, 7, 7]) == [0]
    assert carry_selection([1, 2, 1, 3, 2, 4]) == [0, 1, 3, 5]
    assert carry_selection(list(range(12))) == list(range(8))  # at most eight per launch
    assert carry_selection([5, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14], 8) == [0, 2, 3, 4, 5, 6, 7, 8]
    assert carry_selection([1, 2, 3], limit=2) == [0, 1]
