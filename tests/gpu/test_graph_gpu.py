"""HIP-graph capture of the hot path: a decode layer (grouped GEMVs and the blocked checker,
BF16 and FP8) captured once and replayed several times, with eager work and synchronisation
between replays, reproduces the eager outputs bit for bit on every replay."""

from __future__ import annotations

import pytest
import torch

from pck.cuda import GpuBlockedChecker, check_many, gemv_group, quantize_fp8
from pck.fp import tree_height

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

SHAPES = [("q", 512, 4096), ("k", 128, 4096), ("o", 512, 4096), ("down", 256, 14336)]


@pytest.mark.parametrize("fp8", [False, True])
def test_graph_replays_match_eager(fp8: bool) -> None:
    gen = torch.Generator().manual_seed(11)
    mats = []
    for _, m, n in SHAPES:
        W = (torch.randn(m, n, generator=gen) * 0.02).to(torch.bfloat16).cuda()
        x = torch.randn(n, generator=gen).to(torch.bfloat16).cuda()
        if fp8:
            W = quantize_fp8(W)[0]
        ref = W.to(torch.bfloat16)
        checker = GpuBlockedChecker(ref, 128, tree_height(n, 256, 16 if fp8 else 8), generator=gen)
        mats.append((W, x, checker))

    def step():  # type: ignore[no-untyped-def]
        ys = gemv_group([(W, x) for W, x, _ in mats[:2]], 256) + [
            gemv_group([(W, x)], 256)[0] for W, x, _ in mats[2:]
        ]
        res = check_many([(c, x, y) for (_, x, c), y in zip(mats, ys)])
        return ys, res

    eager_y, eager_res = step()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_y, g_res = step()
    for replay in range(4):
        for y in g_y:
            y.fill_(float("nan"))  # eager work between replays; the replay must overwrite it
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(g_y, eager_y):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32)), replay
        for a, b in zip(g_res, eager_res):
            assert torch.equal(a.passed, b.passed) and a.passed.all()
            assert torch.equal(a.rho, b.rho) and torch.equal(a.tau, b.tau)
