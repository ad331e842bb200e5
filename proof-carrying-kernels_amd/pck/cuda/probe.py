"""Probes of the device arithmetic the error bounds assume (libpck_probe.so, built with the
library's flags; header include/pck_probe.h).  Tests call these on the GPU and compare the
results with exact host arithmetic; nothing in the product path uses them.

Operands are in lane order: for a chain of ``steps`` matrix-core steps over ``tiles`` tiles,
``a`` and ``b`` have shape (tiles, steps, 64) (FP64), (tiles, steps, 64, 8) (BF16, 16 K-slots
per step) or (tiles, steps, 64, 4) (BF16 32x32x8), the accumulator ``c`` (tiles, 64, R) with R
result registers per lane (4 for FP64 16x16x4, 16 for BF16 32x32x16 and 32x32x8, 4 for BF16
16x16x32), and the result has the shape of ``c``.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

from pck.cuda._lib import check, stream_handle

LIBRARY = Path(__file__).resolve().parents[1] / "libpck_probe.so"

_p, _i64, _int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
SIGNATURES = {
    "pck_probe_expf": [_p, _p, _i64, _p],
    "pck_probe_mfma_f64": [_p, _p, _p, _p, _i64, _int, _p],
    "pck_probe_mfma_bf16": [_p, _p, _p, _p, _i64, _int, _p],
    "pck_probe_mfma_bf16_16x16": [_p, _p, _p, _p, _i64, _int, _p],
    "pck_probe_mfma_bf16_k8": [_p, _p, _p, _p, _i64, _int, _p],
    "pck_probe_round_up": [_p, _p, _p, _i64, _p],
    "pck_probe_round_up_mode": [_p, _p, _p, _i64, _p],
}
_handle: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded probe library; raises if it has not been built."""
    global _handle
    if _handle is None:
        if not LIBRARY.exists():
            raise RuntimeError(f"{LIBRARY.name} is not built; run `python -m pck._build` first")
        handle = ctypes.CDLL(str(LIBRARY))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = _int
        _handle = handle
    return _handle


def _cuda(t: torch.Tensor, dtype: torch.dtype, shape: tuple[int, ...], name: str) -> torch.Tensor:
    if not (t.is_cuda and t.dtype == dtype and tuple(t.shape) == shape and t.is_contiguous()):
        raise RuntimeError(f"{name} must be a contiguous {dtype} CUDA tensor of shape {shape}, "
                           f"got {t.dtype} {tuple(t.shape)} on {t.device}")  # fmt: skip
    return t


def expf(x: torch.Tensor) -> torch.Tensor:
    """The device ``expf`` of every element of the FP32 CUDA tensor ``x``."""
    x = _cuda(x, torch.float32, tuple(x.shape), "x")
    y = torch.empty_like(x)
    with torch.cuda.device(x.device):
        check(lib().pck_probe_expf(x.data_ptr(), y.data_ptr(), x.numel(), stream_handle(x.device)),
              "expf probe")  # fmt: skip
    return y


def round_up(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """(n, 4) FP64: the device's mul_up, mul_up_pos, add_up and add_up_nonneg of the FP64 CUDA
    tensors ``a`` and ``b`` (same shape, flattened)."""
    a = _cuda(a, torch.float64, tuple(a.shape), "a")
    b = _cuda(b, torch.float64, tuple(a.shape), "b")
    out = torch.empty((a.numel(), 4), dtype=torch.float64, device=a.device)
    with torch.cuda.device(a.device):
        check(lib().pck_probe_round_up(a.data_ptr(), b.data_ptr(), out.data_ptr(), a.numel(),
                                       stream_handle(a.device)), "round_up probe")  # fmt: skip
    return out


def round_up_mode(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """(n, 3) FP64: the device's add_up_rm2 and add_up_rm4 sums of the FP64 CUDA tensors ``a``
    and ``b`` (same shape, flattened), and an ordinary add issued after them."""
    a = _cuda(a, torch.float64, tuple(a.shape), "a")
    b = _cuda(b, torch.float64, tuple(a.shape), "b")
    out = torch.empty((a.numel(), 3), dtype=torch.float64, device=a.device)
    with torch.cuda.device(a.device):
        check(lib().pck_probe_round_up_mode(a.data_ptr(), b.data_ptr(), out.data_ptr(), a.numel(),
                                            stream_handle(a.device)), "round_up_mode probe")  # fmt: skip
    return out


def _chain(name: str, a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, elems: int,
           regs: int, dtype: torch.dtype) -> torch.Tensor:  # fmt: skip
    if a.dim() < 3:
        raise RuntimeError("a must have shape (tiles, steps, 64[, 8])")
    tiles, steps = a.shape[0], a.shape[1]
    shape = (tiles, steps, 64) + ((elems,) if elems > 1 else ())
    _cuda(a, dtype, shape, "a")
    _cuda(b, dtype, shape, "b")
    acc_dtype = torch.float64 if dtype == torch.float64 else torch.float32
    _cuda(c, acc_dtype, (tiles, 64, regs), "c")
    if not (1 <= tiles <= 1 << 20 and 1 <= steps <= 64):
        raise RuntimeError(f"need 1 <= tiles <= 2^20 and 1 <= steps <= 64, got {tiles}, {steps}")
    d = torch.empty_like(c)
    with torch.cuda.device(c.device):
        err = getattr(lib(), name)(a.data_ptr(), b.data_ptr(), c.data_ptr(), d.data_ptr(), tiles,
                                   steps, stream_handle(c.device))  # fmt: skip
    check(err, name)
    return d


def mfma_f64(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
    """Chains of v_mfma_f64_16x16x4_f64 (a, b: (tiles, steps, 64) FP64; c: (tiles, 64, 4))."""
    return _chain("pck_probe_mfma_f64", a, b, c, 1, 4, torch.float64)


def mfma_bf16(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
    """Chains of v_mfma_f32_32x32x16_bf16 (a, b: (tiles, steps, 64, 8) BF16; c: (tiles, 64, 16)
    FP32)."""
    return _chain("pck_probe_mfma_bf16", a.view(torch.int16), b.view(torch.int16), c, 8, 16,
                  torch.int16)  # fmt: skip


def mfma_bf16_16x16(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
    """Chains of v_mfma_f32_16x16x32_bf16 (a, b: (tiles, steps, 64, 8) BF16; c: (tiles, 64, 4)
    FP32)."""
    return _chain("pck_probe_mfma_bf16_16x16", a.view(torch.int16), b.view(torch.int16), c, 8, 4,
                  torch.int16)  # fmt: skip


def mfma_bf16_k8(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
    """Chains of v_mfma_f32_32x32x8_bf16, the batched product's instruction (a, b: (tiles,
    steps, 64, 4) BF16, lane l + 32 h holding row / column l and K-slots 4h .. 4h + 3;
    c: (tiles, 64, 16) FP32)."""
    return _chain("pck_probe_mfma_bf16_k8", a.view(torch.int16), b.view(torch.int16), c, 4, 16,
                  torch.int16)  # fmt: skip
