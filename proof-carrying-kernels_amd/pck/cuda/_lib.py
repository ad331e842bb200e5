"""ctypes binding of libpck_hip.so (declared in include/pck_hip.h).

The library is the only compute path: if it is missing, every GPU entry point raises instead
of falling back to anything else.  torch is imported before the library is opened so that the
library binds to the HIP runtime torch already loaded (same soname), and torch's stream handles
are valid inside it.
"""

from __future__ import annotations

import ctypes
import functools
from pathlib import Path
from typing import Any

import torch  # noqa: F401  (must be loaded before the library; see the module docstring)

LIBRARY = Path(__file__).resolve().parent.parent / "libpck_hip.so"

MAX_GROUP = 8
MAX_BATCH = 8

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_int = ctypes.c_int
_f64 = ctypes.c_double


class PckGemv(ctypes.Structure):
    _fields_ = [("W", _p), ("x", _p), ("y", _p), ("m", _i64), ("n", _i64)]


class PckCheckDesc(ctypes.Structure):
    _fields_ = [
        ("c", _p),
        ("a", _p),
        ("r", _p),
        ("x", _p),
        ("y", _p),
        ("partial_cx", _p),
        ("partial_s", _p),
        ("counters", _p),
        ("passed", _p),
        ("rho", _p),
        ("tau", _p),
        ("n", _i64),
        ("seg_len", _i64),
        ("block", _i32),
        ("num_blocks", _i32),
        ("checks", _i32),
        ("segments", _i32),
        ("coef", _f64),
        ("geps", _f64),
        ("tau_floor", _f64),
    ]


class PckCheckBatch(ctypes.Structure):
    _fields_ = [
        ("desc", PckCheckDesc * MAX_BATCH),
        ("start", _i64 * (MAX_BATCH + 1)),
        ("count", _i32),
    ]


class PckBatchCheckDesc(ctypes.Structure):
    _fields_ = [
        ("c", _p),
        ("a", _p),
        ("r", _p),
        ("X", _p),
        ("Y", _p),
        ("passed", _p),
        ("rho", _p),
        ("tau", _p),
        ("n", _i64),
        ("block", _i64),
        ("num_blocks", _i64),
        ("checks", _i64),
        ("batch", _i64),
        ("coef", _f64),
        ("geps", _f64),
        ("tau_floor", _f64),
    ]


class PckRowSumCheckDesc(ctypes.Structure):
    _fields_ = [
        ("sums", _p),
        ("y", _p),
        ("r", _p),
        ("passed", _p),
        ("rho", _p),
        ("tau", _p),
        ("block", _i32),
        ("num_blocks", _i32),
        ("checks", _i32),
        ("reserved", _i32),
        ("coef", _f64),
        ("geps", _f64),
        ("tau_floor", _f64),
        ("s_factor", _f64),
    ]


class PckRowSumBatch(ctypes.Structure):
    _fields_ = [
        ("desc", PckRowSumCheckDesc * MAX_BATCH),
        ("start", _i64 * (MAX_BATCH + 1)),
        ("count", _i32),
    ]


class PckMemberArgs(ctypes.Structure):
    _fields_ = [
        ("logits", _p),
        ("rows", _i64),
        ("vocab", _i64),
        ("tokens", _p),
        ("top_k", _p),
        ("top_p", _p),
        ("greedy", _p),
        ("temperature", _p),
        ("temperature_index", _p),
        ("temperature_count", _i64),
        ("injected", _p),
        ("slack", _f64),
        ("k_lim", _i64),
        ("all_k", _i32),
        ("top_p_fp32", _i32),
        ("ok", _p),
        ("above", _p),
        ("mass_above", _p),
        ("totals", _p),
    ]


# name -> (argtypes); every entry point returns int (a hipError_t value)
SIGNATURES: dict[str, list[Any]] = {
    "pck_gemv_bf16_naive": [_p, _p, _p, _i64, _i64, _int, _p],
    "pck_gemv_bf16_coalesced": [_p, _p, _p, _i64, _i64, _int, _p],
    "pck_gemv_fp8_coalesced": [_p, _p, _p, _i64, _i64, _int, _p],
    "pck_gemv_group": [_int, ctypes.POINTER(PckGemv), _int, _int, _p],
    "pck_gemv_group_check": [_int, ctypes.POINTER(PckGemv), _int, _int, _p, _p],
    "pck_gemv_group_fp8_scaled": [ctypes.POINTER(PckGemv), _p, _p, _int, _int, _p, _p],
    "pck_gemv_set_shape": [_int, _int, _int],
    "pck_bgemm": [_int, _p, _p, _p, _i64, _i64, _i64, _p],
    "pck_bgemm_set_shape": [_int, _int],
    "pck_bgemm_pack": [_int, _p, _p, _i64, _i64, _p],
    "pck_bgemm_packed": [_int, _p, _p, _p, _i64, _i64, _i64, _p],
    "pck_blocked_check": [ctypes.POINTER(PckCheckBatch), _p],
    "pck_gemv_group_rowsums": [
        _int, ctypes.POINTER(PckGemv), ctypes.POINTER(_p), _int, _int, _p, _p,
    ],  # fmt: skip
    "pck_rowsum_check": [ctypes.POINTER(PckRowSumBatch), _p],
    "pck_batch_check_workspace": [ctypes.POINTER(PckBatchCheckDesc), _int, ctypes.POINTER(_i64)],
    "pck_batch_check": [ctypes.POINTER(PckBatchCheckDesc), _int, _p, _i64, _p],
    "pck_batch_check_static": [ctypes.POINTER(PckBatchCheckDesc), _int, _p],
    "pck_batch_check_static_init": [],
    "pck_read_stream": [_p, _i64, _p, _int, _p],
    "pck_check_members": [
        _p, _i64, _i64, _p, _p, _p, _p, _f64, _i64, _int, _p, _p, _p, _p,
    ],  # fmt: skip
    "pck_check_members_ex": [ctypes.POINTER(PckMemberArgs), _p],
    "pck_sampling_check": [
        _p, _p, _p, _i64, _i64, _i64, _i64, _int, _f64, _f64, _f64, _i64,
        _p, _p, _p, _p, _p, _p, _p, _p,
    ],  # fmt: skip
}
# size queries, returning int64 (-1 for an invalid argument)
SIZE_QUERIES: dict[str, list[Any]] = {
    "pck_sampling_scratch_words": [_i64],
    "pck_sampling_partial_bytes": [],
    "pck_batch_check_static_bytes": [],
}


@functools.cache
def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    if not LIBRARY.exists():
        raise RuntimeError(
            f"{LIBRARY.name} is not built; run `python -m pck._build` (or "
            "__graft_entry__.build()) first. There is no fallback path."
        )
    handle = ctypes.CDLL(str(LIBRARY))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = argtypes
        fn.restype = _int
    for name, argtypes in SIZE_QUERIES.items():
        fn = getattr(handle, name)
        fn.argtypes = argtypes
        fn.restype = _i64
    handle.pck_sampling_needs_scratch.argtypes = [_i64, _i64, _i64]
    handle.pck_sampling_needs_scratch.restype = _int
    handle.pck_error_string.argtypes = [_int]
    handle.pck_error_string.restype = ctypes.c_char_p
    return handle


def check(err: int, what: str) -> None:
    """Raise RuntimeError for a non-zero hipError_t from the library."""
    if err != 0:
        text = lib().pck_error_string(err).decode()
        raise RuntimeError(f"{what} failed: {text} (hipError_t {err})")


def stream_handle(device: torch.device) -> int:
    """The raw hipStream_t of torch's current stream on ``device``."""
    return int(torch.cuda.current_stream(device).cuda_stream)
