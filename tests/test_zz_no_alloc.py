"""The allocation-free batched checker, `pck_batch_check_static`, through the C-ABI.

- On the GPU its outputs equal `pck_batch_check`'s bit for bit (passed, rho and tau of every
  (check, block, column)) on two calls in a row: a Llama-3-8B decode layer at batch 128 with
  planted faults, then a smaller layer at batch 33 (the second call reuses the device array
  the first one left its partial sums in);
- replays of a HIP graph that captured it equal the eager call, with eager work between,
  also in a fresh process whose first call is the captured one (after
  pck_batch_check_static_init, the lookup of the array's address, outside the capture);
- on the host, with no GPU: a plan beyond the static array returns hipErrorOutOfMemory and an
  invalid descriptor hipErrorInvalidValue, both before any HIP call (the descriptors' pointers
  are never dereferenced there).
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from pck.cuda import GpuBlockedChecker, batched_height, gemm_batched
from pck.cuda._lib import PckBatchCheckDesc, check, lib, stream_handle
from pck.cuda.checker import CheckResult, batched_descriptors

HIP_ERROR_INVALID_VALUE = 1
HIP_ERROR_OUT_OF_MEMORY = 2

gpu = pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")


def layer(shapes: list[tuple[int, int]], B: int, seed: int, faults: bool):  # type: ignore[no-untyped-def]
    """(checker, X, Y) per projection; with ``faults``, the top exponent bit of one output per
    64 rows of column 0 and the sign of every output of column B - 1 in the first block are
    flipped."""
    g = torch.Generator().manual_seed(seed)
    items = []
    for m, n in shapes:
        W = (torch.randn(m, n, generator=g) * 0.02).to(torch.bfloat16).cuda()
        X = torch.randn(B, n, generator=g).to(torch.bfloat16).cuda()
        Y = gemm_batched(W, X)
        if faults:
            bits = Y.view(torch.int32)
            bits[0, ::64] ^= 1 << 30
            bits[B - 1, :128] ^= -(1 << 31)
        checker = GpuBlockedChecker(W, 128, batched_height(n), checks=2,
                                    generator=torch.Generator().manual_seed(m + seed))  # fmt: skip
        items.append((checker, X, Y))
    return items


def with_workspace(items) -> list[CheckResult]:  # type: ignore[no-untyped-def]
    descs, results, device = batched_descriptors(items)
    need = ctypes.c_int64(0)
    check(lib().pck_batch_check_workspace(descs, len(items), ctypes.byref(need)), "plan")
    work = torch.empty(max(1, need.value // 8), dtype=torch.float64, device=device)
    check(lib().pck_batch_check(descs, len(items), work.data_ptr(), need.value,
                                stream_handle(device)), "pck_batch_check")  # fmt: skip
    return results


def without_workspace(items) -> tuple[list[CheckResult], int]:  # type: ignore[no-untyped-def]
    descs, results, device = batched_descriptors(items)
    need = ctypes.c_int64(0)
    check(lib().pck_batch_check_workspace(descs, len(items), ctypes.byref(need)), "plan")
    check(lib().pck_batch_check_static(descs, len(items), stream_handle(device)),
          "pck_batch_check_static")  # fmt: skip
    return results, need.value


def assert_bitwise_equal(got: list[CheckResult], want: list[CheckResult]) -> None:
    assert len(got) == len(want)
    for g, w in zip(got, want, strict=True):
        assert torch.equal(g.passed, w.passed)
        assert torch.equal(g.rho.view(torch.int64), w.rho.view(torch.int64))
        assert torch.equal(g.tau.view(torch.int64), w.tau.view(torch.int64))


LLAMA = [(6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336)]


@pytest.mark.gpu
@gpu
def test_equals_the_workspace_entry_on_two_calls() -> None:
    limit = lib().pck_batch_check_static_bytes()
    assert limit == 16 << 20
    for shapes, B, seed in ((LLAMA, 128, 1), ([(4096, 4096), (1024, 14336)], 33, 2)):
        print(f"static batch check B={B} shapes={shapes}", flush=True)
        items = layer(shapes, B, seed, faults=True)
        got, need = without_workspace(items)
        assert 0 < need <= limit
        want = with_workspace(items)
        torch.cuda.synchronize()
        assert_bitwise_equal(got, want)
        for res in want:  # the faults were planted and are caught; honest columns pass
            assert not bool(res.passed.all())
            assert bool(res.passed[:, :, 1 : B - 1].all())


@pytest.mark.gpu
@gpu
def test_graph_replays_equal_the_eager_call() -> None:
    print("static batch check under graph capture", flush=True)
    items = layer(LLAMA[:2], 64, 3, faults=True)
    want = with_workspace(items)
    descs, results, device = batched_descriptors(items)
    with torch.cuda.device(device):  # the per-device address lookup, outside the capture
        check(lib().pck_batch_check_static_init(), "pck_batch_check_static_init")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        err = lib().pck_batch_check_static(descs, len(items), stream_handle(device))
    check(err, "pck_batch_check_static under capture")
    for replay in range(3):
        for res in results:
            res.rho.fill_(float("nan"))
            res.tau.fill_(float("nan"))
            res.passed.fill_(False)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"replay {replay}", flush=True)
        assert_bitwise_equal(results, want)
        with_workspace(items)  # eager use of the same checker between replays
        torch.cuda.synchronize()


FIRST_CALL_UNDER_CAPTURE = """
import sys, torch
sys.path[:0] = [{root!r}, {root!r} + "/proof-carrying-kernels_amd"]
from tests.test_zz_no_alloc import LLAMA, assert_bitwise_equal, layer, with_workspace
from pck.cuda._lib import check, lib, stream_handle
from pck.cuda.checker import batched_descriptors
items = layer(LLAMA[2:4], 40, 5, faults=True)
want = with_workspace(items)
descs, results, device = batched_descriptors(items)
check(lib().pck_batch_check_static_init(), "init")
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    err = lib().pck_batch_check_static(descs, len(items), stream_handle(device))
check(err, "first pck_batch_check_static call, under capture")
for replay in range(2):
    graph.replay()
    torch.cuda.synchronize()
    assert_bitwise_equal(results, want)
print("first call under capture: replays equal the workspace entry")
"""


@pytest.mark.gpu
@gpu
def test_first_call_of_a_fresh_process_under_capture() -> None:
    """In a fresh process (no earlier call has looked the array up), pck_batch_check_static_init
    and then a first call made under graph capture: every replay equals pck_batch_check."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parent.parent)
    print("fresh process: first static call under capture", flush=True)
    done = subprocess.run([sys.executable, "-c", FIRST_CALL_UNDER_CAPTURE.format(root=root)],
                          capture_output=True, text=True, timeout=110, cwd=root)  # fmt: skip
    print(done.stdout[-2000:], done.stderr[-2000:], flush=True)
    assert done.returncode == 0
    assert "replays equal the workspace entry" in done.stdout


def fake_desc(m: int, n: int, B: int, checks: int) -> PckBatchCheckDesc:
    """A descriptor with aligned stand-in pointers: the host plans it without reading them."""
    block = 128
    return PckBatchCheckDesc(0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 0x6000, 0x7000, 0x8000,
                             n, block, m // block, checks, B, 0.0, 0.0, 0.0)  # fmt: skip


def test_oversized_or_invalid_plans_enqueue_nothing() -> None:
    limit = lib().pck_batch_check_static_bytes()
    # 8 checks at B = 1024: 32 MiB of partial sums
    descs = (PckBatchCheckDesc * 2)(fake_desc(28672, 4096, 1024, 8), fake_desc(4096, 14336, 1024, 8))
    need = ctypes.c_int64(0)
    check(lib().pck_batch_check_workspace(descs, 2, ctypes.byref(need)), "plan")
    assert need.value > limit
    assert lib().pck_batch_check_static(descs, 2, None) == HIP_ERROR_OUT_OF_MEMORY
    bad = (PckBatchCheckDesc * 1)(fake_desc(4096, 4100, 8, 1))  # n % 8 != 0
    assert lib().pck_batch_check_static(bad, 1, None) == HIP_ERROR_INVALID_VALUE
    assert lib().pck_batch_check_static(descs, 0, None) == HIP_ERROR_INVALID_VALUE
