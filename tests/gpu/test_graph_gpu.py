"""HIP-graph capture of the hot path: a decode layer (grouped GEMVs and the blocked checker,
BF16 and FP8), the batched path (packs, packed products, the batched checker), the membership
check and the set-sampling checker, each captured once and replayed several times with eager
work and synchronisation between replays, reproduce the eager outputs bit for bit on every
replay."""

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


def test_batched_layer_graph_replays_match_eager() -> None:
    """The batched path under capture: activation packs, packed products (gate/up at B = 128
    takes two launches, its uneven last round split off) and one batched checker call, BF16
    and FP8 weights; every replay equals the eager run bit for bit, with eager work between."""
    from pck.cuda import batched_height, check_batched, gemm_batched, pack_batched_weights

    gen = torch.Generator().manual_seed(12)
    B = 128
    items = []
    for m, n, fp8 in ((28672, 4096, False), (4096, 14336, True)):
        W = (torch.randn(m, n, generator=gen) * 0.02).to(torch.bfloat16).cuda()
        if fp8:
            W = quantize_fp8(W)[0]
        ref = W.to(torch.bfloat16)
        X = torch.randn(B, n, generator=gen).to(torch.bfloat16).cuda()
        checker = GpuBlockedChecker(ref, 128, batched_height(n), generator=gen)
        items.append((pack_batched_weights(W), X, checker))

    def step():  # type: ignore[no-untyped-def]
        ys = [gemm_batched(Wp, X) for Wp, X, _ in items]
        return ys, check_batched([(c, X, Y) for (_, X, c), Y in zip(items, ys)])

    print("batched layer under graph capture", flush=True)
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
        for r in g_res:
            r.rho.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(g_y, eager_y):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32)), replay
        for a, b in zip(g_res, eager_res):
            assert torch.equal(a.passed, b.passed) and bool(a.passed.all()), replay
            assert torch.equal(a.rho, b.rho) and torch.equal(a.tau, b.tau), replay


def test_membership_graph_replays_match_eager() -> None:
    """The membership check under capture (B = 64, V = 151936, top-k and top-p rows, greedy
    rows, one planted out-of-set token), given the host copy of top-k as vLLM passes it: every
    replay equals the eager run, with eager work between replays."""
    from pck.member import check_members

    gen = torch.Generator().manual_seed(13)
    B, V = 64, 151936
    logits = (torch.randn(B, V, generator=gen) * 3).cuda()
    top_k = torch.randint(1, 200, (B,), generator=gen).cuda()
    top_p = (torch.rand(B, generator=gen) * 0.5 + 0.5).cuda()
    greedy = torch.zeros(B, dtype=torch.bool)
    greedy[::9] = True
    greedy = greedy.cuda()
    tokens = logits.argmax(dim=1)
    tokens[5] = logits[5].argmin()  # outside every set: rejected

    top_k_host = top_k.cpu().numpy()  # a capture cannot copy top-k to the host itself

    def step():  # type: ignore[no-untyped-def]
        return check_members(logits, tokens, top_k=top_k, top_p=top_p, greedy=greedy,
                             top_k_host=top_k_host)  # fmt: skip

    print("membership under graph capture", flush=True)
    eager = step()
    torch.cuda.synchronize()
    assert not bool(eager["ok"][5]) and int(eager["ok"].sum()) == B - 1
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = step()
    for replay in range(4):
        for t in got.values():
            t.zero_()  # eager work between replays; the replay must overwrite it
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for key in ("ok", "above", "mass_above"):
            assert torch.equal(got[key], eager[key]), (key, replay)


def test_set_sampling_checks_graph_replays_match_eager() -> None:
    """The set-sampling checker under capture (top-k and top-p, B = 8, V = 151936, one row's
    top-k set with a swapped member): every replay equals the eager run, with eager work
    between replays."""
    from pck.cuda import check_topk_gpu, check_topp_gpu, topk_sample, topp_select

    gen = torch.Generator().manual_seed(14)
    B, V, k, p = 8, 151936, 50, 0.9
    logits = (torch.randn(B, V, generator=gen) * 2).cuda()
    selected, _ = topk_sample(logits, k)
    selected[3, 0] = logits[3].argmin()  # not a top-k set
    nucleus, lengths = topp_select(logits, p)

    def step():  # type: ignore[no-untyped-def]
        return check_topk_gpu(logits, selected, k), check_topp_gpu(logits, nucleus, lengths, p)

    print("set-sampling checks under graph capture", flush=True)
    eager = step()
    torch.cuda.synchronize()
    assert not bool(eager[0].passed[3]) and int(eager[0].passed.sum()) == B - 1
    assert bool(eager[1].passed.all())
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = step()
    fields = ("passed", "min_selected", "max_rejected", "mass", "mass_without_smallest")
    for replay in range(4):
        for res in got:
            for f in fields:
                getattr(res, f).zero_()  # eager work between replays; the replay must overwrite it
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(got, eager):
            for f in fields:
                assert torch.equal(_bits(getattr(a, f)), _bits(getattr(b, f))), (f, replay)


def _bits(t: torch.Tensor) -> torch.Tensor:
    """The tensor's bit patterns (equal NaNs compare equal)."""
    if t.dtype == torch.float64:
        return t.view(torch.int64)
    return t.view(torch.int32) if t.dtype == torch.float32 else t
