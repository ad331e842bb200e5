"""Host logic of the agent-template wrappers, without a GPU: flag bits, the INT8 copy being
required, and the reference's validation messages for inputs that are not on a GPU."""

from __future__ import annotations

import pytest
import torch

from pck.agent.column import ColumnConfig
from pck.agent.config import KernelConfig, template_flags
from pck.cuda import gemv_column, gemv_template


def test_flag_bits_follow_the_reference() -> None:
    assert template_flags(KernelConfig()) == 0
    assert template_flags(KernelConfig(acc="bf16")) == 1
    assert template_flags(KernelConfig(partials="bf16")) == 2
    assert template_flags(KernelConfig(out="bf16")) == 4
    assert template_flags(KernelConfig(threads=64, skip_tail=True)) == 8


def test_an_int8_config_needs_its_copy() -> None:
    W = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="INT8 copy"):
        gemv_template(W, torch.zeros(64, dtype=torch.bfloat16), KernelConfig(weights="int8"))


def test_host_tensors_are_refused_with_the_reference_messages() -> None:
    W = torch.zeros(4, 64, dtype=torch.bfloat16)
    x = torch.zeros(64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="W and x must be CUDA tensors"):
        gemv_template(W, x, KernelConfig())
    with pytest.raises(RuntimeError, match="rows_per_block must divide threads"):
        from pck.cuda.template import _template

        _template(W, x, 64, 3, 8, 1, 0)
    with pytest.raises(RuntimeError, match="Wq, S and x must be CUDA tensors on one device"):
        gemv_template(W, x, KernelConfig(weights="int8"), (W.to(torch.int8), torch.zeros(4, 1)))
    with pytest.raises(RuntimeError, match="WT and x must be CUDA tensors on one device"):
        gemv_column(W.t().contiguous(), torch.zeros(4, dtype=torch.bfloat16), ColumnConfig())
