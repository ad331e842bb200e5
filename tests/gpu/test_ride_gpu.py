"""Checks carried inside a later GEMV launch (pck_gemv_group_check): rho, tau and verdicts are
bit-identical to the standalone checker on the same items, for BF16 and FP8 launches, padded
and unpadded rows, the fallback configurations (threads != 256, element loads), graph capture,
and a planted fault is caught in the carrying launch exactly as by check_many."""

from __future__ import annotations

import pytest
import torch

from pck.cuda import GpuBlockedChecker, check_many, gemv_group, gemv_group_check, quantize_fp8
from pck.fp import tree_height

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def layer(shapes, seed, fp8=False, threads=256):  # type: ignore[no-untyped-def]
    gen = torch.Generator().manual_seed(seed)
    out = []
    for m, n in shapes:
        W = (torch.randn(m, n, generator=gen) * 0.02).to(torch.bfloat16).cuda()
        x = torch.randn(n, generator=gen).to(torch.bfloat16).cuda()
        if fp8:
            W = quantize_fp8(W)[0]
        vec = 16 if fp8 else 8
        checker = GpuBlockedChecker(W.to(torch.bfloat16), 128, tree_height(n, threads, vec), generator=gen)
        out.append((W, x, checker))
    return out


def same(a, b) -> None:  # type: ignore[no-untyped-def]
    assert torch.equal(a.passed, b.passed)
    assert torch.equal(a.rho, b.rho)
    assert torch.equal(a.tau, b.tau)


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("carrier", [[(4096, 4096)], [(512, 14336)], [(1024, 4096), (1024, 4096)], [(768, 4100)]])
def test_carried_checks_equal_standalone(fp8: bool, carrier) -> None:  # type: ignore[no-untyped-def]
    produced = layer([(1024, 4096), (512, 14336), (256, 4100)], seed=1, fp8=fp8)
    ys = [gemv_group([(W, x)], 256)[0] for W, x, _ in produced]
    items = [(ch, x, y) for (W, x, ch), y in zip(produced, ys)]
    alone = check_many(items)
    carry = layer(carrier, seed=2, fp8=fp8)
    outs, riding = gemv_group_check([(W, x) for W, x, _ in carry], items, 256)
    for a, b in zip(riding, alone):
        same(a, b)
        assert a.verdict.all()
    for (W, x, _), y in zip(carry, outs):  # the carrying GEMVs keep their own bits
        assert torch.equal(y.view(torch.int32), gemv_group([(W, x)], 256)[0].view(torch.int32))


@pytest.mark.parametrize("threads", [128, 512])
def test_fallback_thread_counts_give_the_same_results(threads: int) -> None:
    produced = layer([(512, 4096)], seed=3, threads=threads)
    W, x, ch = produced[0]
    y = gemv_group([(W, x)], threads)[0]
    alone = check_many([(ch, x, y)])
    carry = layer([(256, 4096)], seed=4)
    outs, riding = gemv_group_check([(carry[0][0], carry[0][1])], [(ch, x, y)], threads)
    same(riding[0], alone[0])


def test_a_planted_fault_is_caught_in_the_carrying_launch() -> None:
    produced = layer([(1024, 4096), (512, 14336)], seed=5)
    ys = [gemv_group([(W, x)], 256)[0] for W, x, _ in produced]
    ys[1][300] += 0.5  # one output of block 2 of the second GEMV
    items = [(ch, x, y) for (W, x, ch), y in zip(produced, ys)]
    carry = layer([(4096, 4096)], seed=6)
    _, riding = gemv_group_check([(carry[0][0], carry[0][1])], items, 256)
    assert riding[0].verdict.all()
    verdict = riding[1].verdict
    assert not verdict[300 // 128] and int(verdict.sum()) == 512 // 128 - 1
    for a, b in zip(riding, check_many(items)):
        same(a, b)


def test_carried_checks_in_a_graph() -> None:
    produced = layer([(1024, 4096), (512, 14336)], seed=7)
    carry = layer([(2048, 4096)], seed=8)

    def step():  # type: ignore[no-untyped-def]
        ys = gemv_group([(W, x) for W, x, _ in produced], 256)
        items = [(ch, x, y) for (W, x, ch), y in zip(produced, ys)]
        outs, riding = gemv_group_check([(carry[0][0], carry[0][1])], items, 256)
        return ys, outs, riding

    eager = step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    for _ in range(3):
        for t in captured[0] + captured[1]:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(captured[0] + captured[1], eager[0] + eager[1]):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32))
        for a, b in zip(captured[2], eager[2]):
            same(a, b)
            assert a.verdict.all()
