"""GPU entry points of the decode hot path (reference `src/pck/cuda/__init__.py`), backed by
the gfx950 library libpck_hip.so.  ``pck.cuda`` keeps the reference's module name: on ROCm,
PyTorch's device API is ``torch.cuda``."""

from pck.cuda.batched import BatchedWeights, batched_height, gemm_batched, pack_batched_weights
from pck.cuda.checker import (
    DEFAULT_BLOCK,
    CheckResult,
    GpuBlockedChecker,
    PendingCheck,
    SideStreamChecker,
    check_batched,
    check_many,
    round_up_bf16,
)
from pck.cuda.sampling import (
    SamplingCheck,
    check_topk_gpu,
    check_topp_gpu,
    default_segments,
    sharded_topk_gpu,
    topk_sample,
    topp_select,
)
from pck.cuda.gemv import (
    gemv_coalesced,
    gemv_fp8,
    gemv_group,
    gemv_group_check,
    gemv_naive,
    quantize_fp8,
)
from pck.cuda.template import column_tiles, gemv_column, gemv_template, row_q8, template_flags

__all__ = [
    "DEFAULT_BLOCK",
    "CheckResult",
    "GpuBlockedChecker",
    "PendingCheck",
    "SideStreamChecker",
    "BatchedWeights",
    "batched_height",
    "check_batched",
    "check_many",
    "gemm_batched",
    "pack_batched_weights",
    "gemv_coalesced",
    "gemv_fp8",
    "gemv_group",
    "gemv_group_check",
    "gemv_naive",
    "quantize_fp8",
    "round_up_bf16",
    "SamplingCheck",
    "check_topk_gpu",
    "check_topp_gpu",
    "default_segments",
    "sharded_topk_gpu",
    "topk_sample",
    "topp_select",
    "column_tiles",
    "gemv_column",
    "gemv_template",
    "row_q8",
    "template_flags",
]
