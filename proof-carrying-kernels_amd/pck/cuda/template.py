"""The agent's GEMV templates on the GPU (reference `src/pck/cuda/gemv.py:61-127`), backed by
libpck_hip.so (`include/pck_template.h`).

Same names, arguments and error behaviour as the reference: `gemv_template` runs the
row-major template with a `KernelConfig` (from the INT8 copy ``q8 = (Wq, S)`` when
``cfg.weights == "int8"``), `row_q8` makes that copy, and `gemv_column` runs the column-major
template with a `ColumnConfig` from ``WT = W.t().contiguous()`` (no merge tickets: the grid
splits are merged by a second launch).  Validation messages follow
`src/pck/cuda/csrc/bindings.cpp:85-151` (RuntimeError).  Outputs are FP32 on the input's device;
kernels are enqueued on the current stream without synchronising.

The INT8 copy is made on the GPU (the reference quantizes with NumPy on the CPU); it is the
same copy bit for bit.
"""

from __future__ import annotations

import ctypes
import functools

import numpy as np
import torch

from pck.agent.column import ColumnConfig
from pck.agent.config import GROUP, KernelConfig, template_flags
from pck.cuda._lib import check, lib, stream_handle
from pck.cuda.gemv import INT32_MAX, _validate

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int

# name -> argtypes; each returns int (a hipError_t value), except the int64 size query
SIGNATURES = {
    "pck_gemv_template": [_p, _p, _p, _i64, _i64, _int, _int, _int, _int, _int, _p],
    "pck_gemv_template_q8": [_p, _p, _p, _p, _i64, _i64, _int, _int, _int, _int, _p],
    "pck_gemv_column": [_p, _p, _p, _p, _p, _i64, _i64, _int, _int, _int, ctypes.c_float, _p],
    "pck_quantize_rows_q8": [_p, _int, _p, _p, _i64, _i64, _p],
}


@functools.cache
def _lib() -> ctypes.CDLL:
    """libpck_hip.so with the template entry points' signatures set."""
    handle = lib()
    for name, argtypes in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = argtypes
        fn.restype = _int
    handle.pck_column_tiles.argtypes = [_i64, _int]
    handle.pck_column_tiles.restype = _i64
    return handle


def column_tiles(m: int, vec: int) -> int:
    """Row tiles of the column-major template, ceil(m / (32 vec)) (the tickets it needs)."""
    return int(_lib().pck_column_tiles(m, vec))


def _template(
    W: torch.Tensor, x: torch.Tensor, threads: int, rows_per_block: int, vec: int, unroll: int,
    flags: int,
) -> torch.Tensor:  # fmt: skip
    """The row-major template (reference binding `src/pck/cuda/csrc/bindings.cpp:85-96`)."""
    if not (rows_per_block > 0 and threads % rows_per_block == 0):
        raise RuntimeError("rows_per_block must divide threads")
    _validate(W, x, threads, 32, torch.bfloat16)
    y = torch.empty(W.size(0), dtype=torch.float32, device=W.device)
    if W.size(0) == 0:
        return y
    if W.size(1) == 0:
        raise RuntimeError("n must be positive")
    with torch.cuda.device(W.device):
        err = _lib().pck_gemv_template(
            W.data_ptr(), x.data_ptr(), y.data_ptr(), W.size(0), W.size(1), threads,
            rows_per_block, vec, unroll, flags, stream_handle(W.device),
        )  # fmt: skip
    check(err, "gemv kernel launch")
    return y


def _template_q8(
    Wq: torch.Tensor, S: torch.Tensor, x: torch.Tensor, threads: int, rows_per_block: int,
    vec: int, unroll: int,
) -> torch.Tensor:  # fmt: skip
    """The INT8 template (reference binding `src/pck/cuda/csrc/bindings.cpp:98-125`)."""
    if not (Wq.is_cuda and S.is_cuda and x.is_cuda and Wq.device == x.device == S.device):
        raise RuntimeError("Wq, S and x must be CUDA tensors on one device")
    if not (Wq.dtype == torch.int8 and S.dtype == torch.float32 and x.dtype == torch.bfloat16):
        raise RuntimeError("Wq must be int8, S float32 and x bfloat16")
    if not (Wq.dim() == 2 and x.dim() == 1 and x.size(0) == Wq.size(1)):
        raise RuntimeError("expected Wq of shape (m, n) and x of shape (n,)")
    m, n = Wq.shape
    if not (S.dim() == 2 and S.size(0) == m and S.size(1) == -(-n // GROUP)):
        raise RuntimeError("expected S of shape (m, ceil(n / 128))")
    if not (Wq.is_contiguous() and S.is_contiguous() and x.is_contiguous()):
        raise RuntimeError("Wq, S and x must be contiguous")
    if not (rows_per_block > 0 and threads % rows_per_block == 0):
        raise RuntimeError("rows_per_block must divide threads")
    if m > INT32_MAX:
        raise RuntimeError("too many rows")
    if n == 0:  # an empty sum
        return torch.zeros(m, dtype=torch.float32, device=x.device)
    y = torch.empty(m, dtype=torch.float32, device=x.device)
    if m == 0:
        return y
    with torch.cuda.device(Wq.device):
        err = _lib().pck_gemv_template_q8(
            Wq.data_ptr(), S.data_ptr(), x.data_ptr(), y.data_ptr(), m, n, threads,
            rows_per_block, vec, unroll, stream_handle(Wq.device),
        )  # fmt: skip
    check(err, "template gemv launch")
    return y


def _column_run(
    WT: torch.Tensor, x: torch.Tensor, threads: int, vec: int, splits: int, skip_below: float,
    tickets: torch.Tensor | None = None,
) -> torch.Tensor:  # fmt: skip
    """The column-major template (reference binding `src/pck/cuda/csrc/bindings.cpp:127-151`);
    ``tickets`` is only validated, as the reference does, and never read."""
    if not (WT.is_cuda and x.is_cuda and WT.device == x.device):
        raise RuntimeError("WT and x must be CUDA tensors on one device")
    if not (WT.dtype == torch.bfloat16 and x.dtype == torch.bfloat16):
        raise RuntimeError("WT and x must be bfloat16")
    if not (WT.dim() == 2 and x.dim() == 1 and x.size(0) == WT.size(0)):
        raise RuntimeError("expected WT of shape (n, m) and x of shape (n,)")
    if not (WT.is_contiguous() and x.is_contiguous()):
        raise RuntimeError("WT and x must be contiguous")
    n, m = WT.shape
    y = torch.empty(m, dtype=torch.float32, device=WT.device)
    scratch = torch.empty(splits * m if splits > 1 else 0, dtype=torch.float32, device=WT.device)
    if m == 0:
        return y
    if tickets is not None:
        tiles = column_tiles(m, vec) if vec in (2, 4, 8) else 0
        if not (
            vec > 0 and tickets.is_cuda and tickets.device == WT.device
            and tickets.dtype == torch.int32 and tickets.is_contiguous() and tickets.numel() >= tiles
        ):  # fmt: skip
            raise RuntimeError(
                "tickets must be a zeroed int32 CUDA tensor with at least one entry per tile"
            )
    with torch.cuda.device(WT.device):
        err = _lib().pck_gemv_column(
            WT.data_ptr(), x.data_ptr(), y.data_ptr(), scratch.data_ptr(), None, m, n, threads,
            vec, splits, skip_below, stream_handle(WT.device),
        )  # fmt: skip
    check(err, "column gemv launch")
    return y


def _column(
    WT: torch.Tensor, x: torch.Tensor, tickets: torch.Tensor, threads: int, vec: int, splits: int,
    skip_below: float,
) -> torch.Tensor:  # fmt: skip
    """The reference extension's signature, with its merge tickets (validated, not read)."""
    return _column_run(WT, x, threads, vec, splits, skip_below, tickets)


def gemv_template(
    W: torch.Tensor,
    x: torch.Tensor,
    cfg: KernelConfig,
    q8: tuple[torch.Tensor, torch.Tensor] | None = None,
) -> torch.Tensor:
    """y = W x with the row-major template instantiated with ``cfg``; with
    ``cfg.weights == "int8"`` from ``q8 = (Wq, S)``, the INT8 copy made by `row_q8`.

    Bit-identical to the template's CPU model for every config.
    """
    if cfg.weights == "int8":
        if q8 is None:
            raise ValueError("an INT8 config needs the INT8 copy of W (q8)")
        return _template_q8(*q8, x, cfg.threads, cfg.rows_per_block, cfg.vec, cfg.unroll)
    return _template(
        W, x, cfg.threads, cfg.rows_per_block, cfg.vec, cfg.unroll, template_flags(cfg)
    )


def row_q8(
    W: np.ndarray | torch.Tensor, device: torch.device | str = "cuda"
) -> tuple[torch.Tensor, torch.Tensor]:
    """The INT8 copy (Wq, S) of W for `gemv_template`, made on ``device``: per row and group of
    128 columns, S = max |w| / 127 (1 for an all-zero group) and Wq = round-half-even(w / S)
    clipped to [-127, 127].  W is taken as FP32 (BF16 tensors as they are) and must be finite.
    """
    if isinstance(W, torch.Tensor):
        Wd = W.to(device)
        if Wd.dtype not in (torch.bfloat16, torch.float32):
            Wd = Wd.float()
    else:
        Wd = torch.from_numpy(np.asarray(W, dtype=np.float32)).to(device)
    Wd = Wd.contiguous()
    if Wd.dim() != 2 or not Wd.is_cuda:
        raise RuntimeError("expected W of shape (m, n) on a CUDA device")
    m, n = Wd.shape
    Wq = torch.empty((m, n), dtype=torch.int8, device=Wd.device)
    S = torch.empty((m, -(-n // GROUP)), dtype=torch.float32, device=Wd.device)
    with torch.cuda.device(Wd.device):
        err = _lib().pck_quantize_rows_q8(
            Wd.data_ptr(), 0 if Wd.dtype == torch.bfloat16 else 1, Wq.data_ptr(), S.data_ptr(),
            m, n, stream_handle(Wd.device),
        )  # fmt: skip
    check(err, "row_q8 kernel launch")
    return Wq, S


def gemv_column(WT: torch.Tensor, x: torch.Tensor, cfg: ColumnConfig) -> torch.Tensor:
    """y = W x with the column-major template, from ``WT = W.t().contiguous()``.

    Bit-identical to the template's CPU model.  The grid splits are merged by a second launch
    on the same stream (no shared tickets), so calls may overlap on one device.
    """
    return _column_run(WT, x, cfg.threads, cfg.vec, cfg.splits, cfg.skip_below)
